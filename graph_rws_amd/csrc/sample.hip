// Node-wise fanout sampling and unique-and-relabel (gfx950).
//
// The reference samples whole row windows with a score top-K
// (core/include/sampling.cuh:65-448, driven by
// core/wrapper/sampling_wrapper.cu:365-438); the mini-batch path of the
// benchmark configuration instead draws a fixed fanout per node, without
// replacement, from a counter-based stream, and relabels the sampled sources
// to the "destination nodes first" local ids that the reference's block
// layers expect (data/bcsr.py:266-306, layers/layer.py:159-161).
//
// Random stream: word 0 of Philox4x32-10 (Salmon et al., SC'11) with
//   key     = (seed_lo, seed_hi)
//   counter = (node_lo, node_hi, draw, 0),
// mapped to [0, m) by the multiply-shift (u64(u) * m) >> 32 (m < 2^32).
//
// One hop (grws_sample_hop): one wave64 per frontier node.  deg <= k takes
// every neighbour; otherwise Floyd's algorithm over j = deg-k .. deg-1 with
// draw index d = j - (deg-k): lane d computes its candidate t_d from its own
// draw (the draws do not depend on earlier choices), then the k choices are
// resolved in order with one ballot each ("t_d already chosen" -> take j_d),
// and the chosen CSR positions are ranked ascending across the wave.  Edges
// are emitted in frontier order, then ascending CSR position, at offsets
// from an exclusive scan of min(deg, k).
//
// Relabel (grws_relabel): frontier nodes keep local ids [0, F) in frontier
// order; sources outside the frontier get F, F+1, ... in ascending global id.
// Both id lists are radix sorted (sort.hip); each sorted source finds its
// frontier position by binary search, first occurrences of new ids are
// ranked by a scan, and the local id is scattered back to the edge.
#include "grws_internal.h"

namespace grws {
namespace {

constexpr int kBlk = 256;
constexpr int kWavesPerBlock = kBlk / kWave;

enum : int32_t { kErrNode = 1, kErrIndptr = 2, kErrIndex = 4, kErrDup = 8, kErrDegree = 16 };

inline int bits_for(int64_t x) {
    int b = 0;
    while (b < 63 && ((int64_t)1 << b) < x) ++b;
    return b;
}

inline unsigned grid_for(int64_t n, int64_t per_block = kBlk) {
    int64_t g = (n + per_block - 1) / per_block;
    return (unsigned)(g < 1 ? 1 : g);
}

__device__ __forceinline__ uint32_t philox_word0(uint64_t seed, uint64_t node, uint32_t draw) {
    uint32_t c0 = (uint32_t)node, c1 = (uint32_t)(node >> 32), c2 = draw, c3 = 0u;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(0xD2511F53u, c0);
        const uint32_t lo0 = 0xD2511F53u * c0;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2);
        const uint32_t lo1 = 0xCD9E8D57u * c2;
        const uint32_t n0 = hi1 ^ c1 ^ k0;
        const uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Validity of one frontier node's neighbour range; both kernels of a hop
// decide identically so the scan's offsets match what the sampler writes.
struct NodeRange {
    int64_t start, deg;
    int32_t err;
};

__device__ __forceinline__ NodeRange node_range(const int64_t* __restrict__ indptr, int64_t nnz, int64_t num_nodes,
                                                int64_t v) {
    NodeRange r{0, 0, 0};
    if (v < 0 || v >= num_nodes) {
        r.err = kErrNode;
        return r;
    }
    const int64_t s = indptr[v], e = indptr[v + 1];
    if (s < 0 || e < s || e > nnz) {
        r.err = kErrIndptr;
        return r;
    }
    if (e - s > (int64_t)UINT32_MAX) {
        r.err = kErrDegree;
        return r;
    }
    r.start = s;
    r.deg = e - s;
    return r;
}

__global__ void hop_count_kernel(const int64_t* __restrict__ indptr, int64_t nnz, int64_t num_nodes,
                                 const int64_t* __restrict__ frontier, int64_t F, int k, int32_t* __restrict__ cnt,
                                 int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= F) return;
    const NodeRange r = node_range(indptr, nnz, num_nodes, frontier[i]);
    if (r.err) atomicOr(err, r.err);
    cnt[i] = (int32_t)(r.deg < k ? r.deg : k);
}

// GCN weight of a sampled edge from full-graph out-degrees:
// 1 / sqrt((deg_dst + 1) (deg_src + 1)), evaluated in double (the product is
// exact, sqrt and division are correctly rounded) and rounded once to float.
__device__ __forceinline__ float gcn_weight(int64_t deg_dst, int64_t deg_src) {
    const double p = (double)(deg_dst + 1) * (double)(deg_src + 1);
    return (float)(1.0 / sqrt(p));
}

__global__ __launch_bounds__(kBlk) void hop_sample_kernel(const int64_t* __restrict__ indptr,
                                                          const int32_t* __restrict__ indices, int64_t nnz,
                                                          int64_t num_nodes, const int64_t* __restrict__ frontier,
                                                          int64_t F, int k, uint64_t seed,
                                                          const int64_t* __restrict__ off,
                                                          int32_t* __restrict__ edge_dst,
                                                          int64_t* __restrict__ edge_src,
                                                          float* __restrict__ edge_val, int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    if (i >= F) return;  // wave-uniform
    const int lane = lane_id();
    const int64_t v = frontier[i];
    const NodeRange r = node_range(indptr, nnz, num_nodes, v);
    if (r.err) return;  // counted as 0 edges by hop_count_kernel
    const int64_t deg = r.deg;
    int64_t x = lane;  // chosen CSR position (relative to r.start)
    int rank = lane;   // its rank among the chosen positions
    int n;
    if (deg <= k) {
        n = (int)deg;
    } else {
        n = k;
        const int64_t j0 = deg - k;
        int64_t t = 0;
        if (lane < k) {
            const uint32_t u = philox_word0(seed, (uint64_t)v, (uint32_t)lane);
            t = (int64_t)(((uint64_t)u * (uint64_t)(j0 + lane + 1)) >> 32);
        }
        // Floyd, in draw order: lanes e < d hold the choices x_e made so far.
        x = -1;
        for (int d = 0; d < k; ++d) {
            const int64_t td = readlane64(t, d);
            const bool taken = __ballot(lane < d && x == td) != 0ull;
            if (lane == d) x = taken ? j0 + d : td;
        }
        rank = 0;
        for (int e = 0; e < k; ++e) rank += readlane64(x, e) < x ? 1 : 0;
    }
    if (lane < n) {
        const int32_t s = indices[r.start + x];
        const int64_t o = off[i] + rank;
        edge_dst[o] = (int32_t)i;
        edge_src[o] = (int64_t)s;
        if (edge_val) {
            float w = 0.0f;
            if (s >= 0 && (int64_t)s < num_nodes) {
                w = gcn_weight(deg, indptr[(int64_t)s + 1] - indptr[s]);
            } else {
                atomicOr(err, kErrIndex);
            }
            edge_val[o] = w;
        } else if (s < 0 || (int64_t)s >= num_nodes) {
            atomicOr(err, kErrIndex);
        }
    }
}

// --- relabel ----------------------------------------------------------------
__global__ void ids_to_keys_kernel(const int64_t* __restrict__ ids, int64_t n, int64_t num_nodes,
                                   uint64_t* __restrict__ keys, uint32_t* __restrict__ pos,
                                   int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t v = ids[i];
    if (v < 0 || v >= num_nodes) {
        atomicOr(err, kErrNode);
        v = 0;
    }
    keys[i] = (uint64_t)v;
    pos[i] = (uint32_t)i;
}

__global__ void dup_check_kernel(const uint64_t* __restrict__ keys, int64_t n, int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0 || i >= n) return;
    if (keys[i] == keys[i - 1]) atomicOr(err, kErrDup);
}

// Position of `key` in the sorted frontier keys, or -1.
__device__ __forceinline__ int64_t find_sorted(const uint64_t* __restrict__ a, int64_t n, uint64_t key) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (a[mid] < key) lo = mid + 1;
        else hi = mid;
    }
    return (lo < n && a[lo] == key) ? lo : -1;
}

__global__ void relabel_flag_kernel(const uint64_t* __restrict__ ekeys, int64_t E,
                                    const uint64_t* __restrict__ fkeys, const uint32_t* __restrict__ fpos, int64_t F,
                                    int32_t* __restrict__ newflag, int32_t* __restrict__ flocal) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= E) return;
    const uint64_t key = ekeys[i];
    const int64_t f = find_sorted(fkeys, F, key);
    if (f >= 0) {
        flocal[i] = (int32_t)fpos[f];
        newflag[i] = 0;
    } else {
        flocal[i] = -1;
        newflag[i] = (i == 0 || ekeys[i - 1] != key) ? 1 : 0;
    }
}

__global__ void relabel_assign_kernel(const uint64_t* __restrict__ ekeys, const uint32_t* __restrict__ eidx,
                                      int64_t E, int64_t F, const int32_t* __restrict__ newflag,
                                      const int32_t* __restrict__ flocal, const int64_t* __restrict__ nrank,
                                      int32_t* __restrict__ src_local, int64_t* __restrict__ next_frontier) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= E) return;
    const int32_t fl = flocal[i];
    int64_t local;
    if (fl >= 0) {
        local = fl;
    } else {
        // inclusive rank of this id's first occurrence among the new ids
        local = F + nrank[i] + newflag[i] - 1;
        if (newflag[i]) next_frontier[local] = (int64_t)ekeys[i];
    }
    src_local[eidx[i]] = (int32_t)local;
}

__global__ void copy_i64_kernel(const int64_t* __restrict__ a, int64_t n, int64_t* __restrict__ b) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) b[i] = a[i];
}

int report(int32_t e, const char* who) {
    if (e & kErrNode) return set_error(GRWS_E_RANGE, "%s: a node id is outside [0, num_nodes)", who);
    if (e & kErrIndptr) return set_error(GRWS_E_RANGE, "%s: indptr is not a valid CSR row pointer", who);
    if (e & kErrIndex) return set_error(GRWS_E_RANGE, "%s: a neighbour index is outside [0, num_nodes)", who);
    if (e & kErrDegree) return set_error(GRWS_E_RANGE, "%s: a node has 2^32 or more neighbours", who);
    if (e & kErrDup) return set_error(GRWS_E_INVALID, "%s: the frontier holds a node id twice", who);
    return GRWS_OK;
}

struct RelabelWs {
    uint64_t *fk, *fk2, *ek, *ek2;
    uint32_t *fp, *fp2, *ep, *ep2;
    int32_t *newflag, *flocal, *err;
    int64_t* nrank;
    char* sort_ws;
    size_t sort_bytes;
    char* scan_ws;
    size_t scan_bytes;
};

template <typename C>
void carve_relabel(C& cv, int64_t F, int64_t E, RelabelWs* w) {
    const int64_t f = F > 0 ? F : 1, e = E > 0 ? E : 1;
    w->fk = cv.template take<uint64_t>(f);
    w->fk2 = cv.template take<uint64_t>(f);
    w->fp = cv.template take<uint32_t>(f);
    w->fp2 = cv.template take<uint32_t>(f);
    w->ek = cv.template take<uint64_t>(e);
    w->ek2 = cv.template take<uint64_t>(e);
    w->ep = cv.template take<uint32_t>(e);
    w->ep2 = cv.template take<uint32_t>(e);
    w->newflag = cv.template take<int32_t>(e);
    w->flocal = cv.template take<int32_t>(e);
    w->nrank = cv.template take<int64_t>(e + 1);
    w->err = cv.template take<int32_t>(64);
    w->sort_bytes = radix_sort_workspace_bytes(f > e ? f : e);
    w->sort_ws = cv.template take<char>(w->sort_bytes);
    w->scan_bytes = scan_workspace_bytes(e);
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

}  // namespace
}  // namespace grws

using namespace grws;

// ---------------------------------------------------------------------------
// one hop of fanout sampling
// ---------------------------------------------------------------------------
extern "C" size_t grws_sample_hop_workspace_bytes(int64_t num_frontier) {
    if (num_frontier < 0) return 0;
    Sizer s;
    s.take<int32_t>((size_t)num_frontier + 1);
    s.take<int64_t>((size_t)num_frontier + 2);
    s.take<int32_t>(64);
    s.used += scan_workspace_bytes(num_frontier) + 256;
    return s.used;
}

extern "C" int grws_sample_hop(const int64_t* indptr, const int32_t* indices, int64_t num_nodes, int64_t nnz,
                               const int64_t* frontier, int64_t num_frontier, int32_t fanout, uint64_t seed,
                               int32_t* edge_dst, int64_t* edge_src, float* edge_val, int64_t edge_capacity,
                               void* workspace, size_t workspace_bytes, int64_t* num_edges_out, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(num_nodes >= 0 && nnz >= 0 && num_frontier >= 0, "sample_hop: negative size");
    GRWS_CHECK_ARG(fanout >= 1 && fanout <= kWave, "sample_hop: fanout must be in [1, 64] (got %d)", fanout);
    GRWS_CHECK_ARG(num_edges_out != nullptr, "sample_hop: null num_edges_out");
    GRWS_CHECK_ARG(edge_capacity >= num_frontier * (int64_t)fanout,
                   "sample_hop: edge_capacity %lld < num_frontier * fanout = %lld", (long long)edge_capacity,
                   (long long)(num_frontier * (int64_t)fanout));
    *num_edges_out = 0;
    if (num_frontier == 0) return GRWS_OK;
    GRWS_CHECK_ARG(indptr && frontier && edge_dst && edge_src, "sample_hop: null pointer");
    if (nnz > 0) GRWS_CHECK_ARG(indices != nullptr, "sample_hop: null indices");
    Carver cv(workspace, workspace_bytes);
    int32_t* cnt = cv.take<int32_t>(num_frontier + 1);
    int64_t* off = cv.take<int64_t>(num_frontier + 2);
    int32_t* err = cv.take<int32_t>(64);
    const size_t scan_bytes = scan_workspace_bytes(num_frontier);
    char* scan_ws = cv.take<char>(scan_bytes);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "sample_hop: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    GRWS_TRY(fill_i32(err, 1, 0, stream));
    hipLaunchKernelGGL(hop_count_kernel, dim3(grid_for(num_frontier)), dim3(kBlk), 0, stream, indptr, nnz, num_nodes,
                       frontier, num_frontier, (int)fanout, cnt, err);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(cnt, off, num_frontier, false, scan_ws, scan_bytes, stream));
    hipLaunchKernelGGL(hop_sample_kernel, dim3(grid_for(num_frontier, kWavesPerBlock)), dim3(kBlk), 0, stream,
                       indptr, indices, nnz, num_nodes, frontier, num_frontier, (int)fanout, seed, off, edge_dst,
                       edge_src, edge_val, err);
    GRWS_LAUNCH_CHECK();
    int64_t E = 0;
    int32_t e = 0;
    GRWS_HIP(hipMemcpyAsync(&E, off + num_frontier, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&e, err, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    GRWS_TRY(report(e, "sample_hop"));
    *num_edges_out = E;
    return GRWS_OK;
}

// ---------------------------------------------------------------------------
// unique + relabel
// ---------------------------------------------------------------------------
extern "C" size_t grws_relabel_workspace_bytes(int64_t num_frontier, int64_t num_edges) {
    if (num_frontier < 0 || num_edges < 0) return 0;
    NullCarver nc;
    RelabelWs w;
    carve_relabel(nc, num_frontier, num_edges, &w);
    return nc.s.used + 256;
}

extern "C" int grws_relabel(const int64_t* frontier, int64_t num_frontier, const int64_t* edge_src, int64_t num_edges,
                            int64_t num_nodes, int32_t* src_local, int64_t* next_frontier, int64_t next_capacity,
                            void* workspace, size_t workspace_bytes, int64_t* num_src_out, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    const int64_t F = num_frontier, E = num_edges;
    GRWS_CHECK_ARG(F >= 0 && E >= 0 && num_nodes >= 0, "relabel: negative size");
    GRWS_CHECK_ARG(F <= INT32_MAX && E <= (int64_t)UINT32_MAX, "relabel: too many ids");
    GRWS_CHECK_ARG(num_src_out != nullptr, "relabel: null num_src_out");
    GRWS_CHECK_ARG(next_capacity >= F + E, "relabel: next_capacity %lld < num_frontier + num_edges = %lld",
                   (long long)next_capacity, (long long)(F + E));
    *num_src_out = 0;
    if (F + E == 0) return GRWS_OK;
    GRWS_CHECK_ARG(next_frontier != nullptr, "relabel: null next_frontier");
    if (F > 0) GRWS_CHECK_ARG(frontier != nullptr, "relabel: null frontier");
    if (E > 0) GRWS_CHECK_ARG(edge_src && src_local, "relabel: null edge arrays");
    Carver cv(workspace, workspace_bytes);
    RelabelWs w;
    carve_relabel(cv, F, E, &w);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "relabel: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const int bits = bits_for(num_nodes);
    GRWS_TRY(fill_i32(w.err, 1, 0, stream));

    // sorted frontier (id -> frontier position), duplicates rejected
    const uint64_t* fk = w.fk;
    const uint32_t* fp = w.fp;
    if (F > 0) {
        hipLaunchKernelGGL(ids_to_keys_kernel, dim3(grid_for(F)), dim3(kBlk), 0, stream, frontier, F, num_nodes, w.fk,
                           w.fp, w.err);
        GRWS_LAUNCH_CHECK();
        bool alt = false;
        GRWS_TRY(radix_sort_pairs(w.fk, w.fp, w.fk2, w.fp2, F, bits, w.sort_ws, w.sort_bytes, stream, &alt));
        fk = alt ? w.fk2 : w.fk;
        fp = alt ? w.fp2 : w.fp;
        hipLaunchKernelGGL(dup_check_kernel, dim3(grid_for(F)), dim3(kBlk), 0, stream, fk, F, w.err);
        GRWS_LAUNCH_CHECK();
        hipLaunchKernelGGL(copy_i64_kernel, dim3(grid_for(F)), dim3(kBlk), 0, stream, frontier, F, next_frontier);
        GRWS_LAUNCH_CHECK();
    }
    int64_t n_new = 0;
    if (E > 0) {
        hipLaunchKernelGGL(ids_to_keys_kernel, dim3(grid_for(E)), dim3(kBlk), 0, stream, edge_src, E, num_nodes, w.ek,
                           w.ep, w.err);
        GRWS_LAUNCH_CHECK();
        bool alt = false;
        GRWS_TRY(radix_sort_pairs(w.ek, w.ep, w.ek2, w.ep2, E, bits, w.sort_ws, w.sort_bytes, stream, &alt));
        const uint64_t* ek = alt ? w.ek2 : w.ek;
        const uint32_t* ep = alt ? w.ep2 : w.ep;
        hipLaunchKernelGGL(relabel_flag_kernel, dim3(grid_for(E)), dim3(kBlk), 0, stream, ek, E, fk, fp, F, w.newflag,
                           w.flocal);
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(scan_i32_to_i64(w.newflag, w.nrank, E, false, w.scan_ws, w.scan_bytes, stream));
        hipLaunchKernelGGL(relabel_assign_kernel, dim3(grid_for(E)), dim3(kBlk), 0, stream, ek, ep, E, F, w.newflag,
                           w.flocal, w.nrank, src_local, next_frontier);
        GRWS_LAUNCH_CHECK();
        GRWS_HIP(hipMemcpyAsync(&n_new, w.nrank + E, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    }
    int32_t e = 0;
    GRWS_HIP(hipMemcpyAsync(&e, w.err, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    GRWS_TRY(report(e, "relabel"));
    *num_src_out = F + n_new;
    return GRWS_OK;
}
