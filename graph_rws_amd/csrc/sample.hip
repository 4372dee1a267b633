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
        // one 32x32->64 multiply each (v_mad_u64_u32)
        const uint64_t m0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t m1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t hi0 = (uint32_t)(m0 >> 32), lo0 = (uint32_t)m0;
        const uint32_t hi1 = (uint32_t)(m1 >> 32), lo1 = (uint32_t)m1;
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


// ---------------------------------------------------------------------------
// fused hop (grws_sample_block): dense relabel + per-window BCSR build
// ---------------------------------------------------------------------------
// node_map[v] is the local id of frontier node v during a call and -1
// otherwise; bitmap bit v marks a new source.  Both are caller-owned state
// that every call leaves as it found it (all -1 / all 0).

// Edge slots at or past the device-side edge count *E read -1.
__global__ void tail_fill_kernel(const int64_t* __restrict__ E, int64_t* __restrict__ edge_src, int64_t cap) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < cap && i >= *E) edge_src[i] = -1;
}

__global__ void map_frontier_kernel(const int64_t* __restrict__ frontier, int64_t F, int64_t num_nodes,
                                    int32_t* __restrict__ node_map, int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= F) return;
    const int64_t v = frontier[i];
    if (v < 0 || v >= num_nodes) {
        atomicOr(err, kErrNode);
        return;
    }
    if (atomicExch(&node_map[v], (int32_t)i) != -1) atomicOr(err, kErrDup);
}

__global__ void mark_new_kernel(const int64_t* __restrict__ edge_src, int64_t E, int64_t num_nodes,
                                const int32_t* __restrict__ node_map, uint32_t* __restrict__ bitmap) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int64_t s = edge_src[e];
    if (s < 0 || s >= num_nodes) return;  // flagged by the sampler
    if (node_map[s] < 0) atomicOr(&bitmap[s >> 5], 1u << (s & 31));
}

__global__ void word_popcount_kernel(const uint32_t* __restrict__ bitmap, int64_t nwords, int32_t* __restrict__ cnt) {
    const int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (w < nwords) cnt[w] = __popc(bitmap[w]);
}

__global__ void assign_local_kernel(const int64_t* __restrict__ edge_src, int64_t E, int64_t num_nodes, int64_t F,
                                    const int32_t* __restrict__ node_map, const uint32_t* __restrict__ bitmap,
                                    const int64_t* __restrict__ wprefix, int32_t* __restrict__ src_local,
                                    int64_t* __restrict__ next_frontier) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int64_t s = edge_src[e];
    if (s < 0 || s >= num_nodes) {
        src_local[e] = 0;
        return;
    }
    const int32_t l = node_map[s];
    if (l >= 0) {
        src_local[e] = l;
        return;
    }
    const int64_t w = s >> 5;
    const uint32_t below = bitmap[w] & ((1u << (s & 31)) - 1u);
    const int64_t local = F + wprefix[w] + __popc(below);
    src_local[e] = (int32_t)local;
    next_frontier[local] = s;  // every edge of this source writes the same value
}

__global__ void reset_state_kernel(const int64_t* __restrict__ frontier, int64_t F,
                                   const int64_t* __restrict__ edge_src, int64_t E, int64_t num_nodes,
                                   int32_t* __restrict__ node_map, uint32_t* __restrict__ bitmap) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < F) {
        const int64_t v = frontier[i];
        if (v >= 0 && v < num_nodes) node_map[v] = -1;
    }
    if (i < E) {
        const int64_t s = edge_src[i];
        if (s >= 0 && s < num_nodes) bitmap[s >> 5] = 0u;
    }
}

__global__ void fill_state_kernel(int32_t* __restrict__ node_map, int64_t n, uint32_t* __restrict__ bitmap,
                                  int64_t nwords) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n || i < nwords; i += stride) {
        if (i < n) node_map[i] = -1;
        if (i < nwords) bitmap[i] = 0u;
    }
}

template <typename VT>
__device__ __forceinline__ VT cvt_value(float v);
template <>
__device__ __forceinline__ float cvt_value<float>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 cvt_value<_Float16>(float v) { return (_Float16)v; }
template <>
__device__ __forceinline__ __hip_bfloat16 cvt_value<__hip_bfloat16>(float v) { return __float2bfloat16(v); }

constexpr int kWinEdges = 1024;  // 16 rows x fanout <= 64

// One work-group per 16-row window of the hop's block.  Its edges are the
// contiguous range [off[16w], off[16w+16]) (rows are frontier positions), at
// most 16 x fanout of them: they are sorted in LDS by (column, row, input
// order), the distinct columns numbered, and -- in the fill pass -- the
// window's tiles written: columns -1 padded, each (row, column) value taken
// from its last edge in input order (the builder's duplicate rule).
template <typename VT>
__global__ __launch_bounds__(256) void block_window_kernel(int fill, const int64_t* __restrict__ off, int64_t F,
                                                           const int32_t* __restrict__ src_local,
                                                           const float* __restrict__ edge_val, int tc,
                                                           int32_t* __restrict__ wtiles,
                                                           const int64_t* __restrict__ window_offset,
                                                           int32_t* __restrict__ out_cols,
                                                           VT* __restrict__ out_vals) {
    __shared__ uint64_t key[kWinEdges];
    __shared__ int64_t roff[17];
    __shared__ int32_t pos[kWinEdges];
    __shared__ int64_t scan_tmp[kBlk / kWave + 1];
    const int tid = threadIdx.x;
    const int64_t w = blockIdx.x;
    const int64_t r0 = w * 16;
    const int64_t r1 = r0 + 16 < F ? r0 + 16 : F;
    if (tid <= 16) roff[tid] = off[r0 + tid < r1 ? r0 + tid : r1];
    __syncthreads();
    const int64_t e0 = roff[0];
    const int n = (int)(roff[16] - e0);  // <= kWinEdges (fanout <= 64)
    int P = 1;
    while (P < n) P <<= 1;
    for (int i = tid; i < P; i += kBlk) {
        uint64_t k = ~0ull;
        if (i < n) {
            int r = 0;
            while (r < 15 && roff[r + 1] <= e0 + i) ++r;
            const uint64_t col = (uint32_t)src_local[e0 + i];
            k = (col << 14) | ((uint64_t)r << 10) | (uint64_t)i;
        }
        key[i] = k;
    }
    __syncthreads();
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < P; i += kBlk) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = (i & size) == 0;
                    const uint64_t a = key[i], b = key[j];
                    if ((a > b) == up) {
                        key[i] = b;
                        key[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    // number the distinct columns: 4 consecutive keys per thread, block scan
    int flags = 0, cnt = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = tid * 4 + q;
        const bool f = i < n && (i == 0 || (key[i] >> 14) != (key[i - 1] >> 14));
        flags |= (f ? 1 : 0) << q;
        cnt += f ? 1 : 0;
    }
    int64_t total;
    const int64_t incl = block_incl_scan<kBlk>(cnt, scan_tmp, &total);
    int run = (int)(incl - cnt);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = tid * 4 + q;
        if (i < n) {
            run += (flags >> q) & 1;
            pos[i] = run - 1;
        }
    }
    const int64_t tiles = (total + tc - 1) / tc;
    if (!fill) {
        if (tid == 0) wtiles[w] = (int32_t)tiles;
        return;
    }
    __syncthreads();
    const int64_t wo = window_offset[w];
    for (int64_t i = tid; i < tiles * tc; i += kBlk) out_cols[wo * tc + i] = -1;
    for (int64_t i = tid; i < tiles * 16 * tc; i += kBlk) out_vals[wo * 16 * tc + i] = cvt_value<VT>(0.0f);
    __syncthreads();
    for (int i = tid; i < n; i += kBlk) {
        const uint64_t k = key[i];
        const int p = pos[i];
        const int64_t tile = wo + p / tc;
        const int c = p % tc;
        if (i == 0 || (key[i - 1] >> 14) != (k >> 14)) out_cols[tile * tc + c] = (int32_t)(k >> 14);
        if (i == n - 1 || (key[i + 1] >> 10) != (k >> 10)) {
            const int r = (int)((k >> 10) & 15u);
            out_vals[(tile * 16 + r) * tc + c] = cvt_value<VT>(edge_val[e0 + (int64_t)(k & 1023u)]);
        }
    }
}

struct BlockWs {
    int32_t* cnt;
    int64_t* off;
    int32_t* err;
    int32_t* edge_dst;
    int64_t* edge_src;
    float* edge_val;
    int32_t* src_local;
    int32_t* wcnt;
    int64_t* wprefix;
    int32_t* wtiles;
    char* scan_ws;
    size_t scan_bytes;
};

template <typename C>
void carve_block(C& cv, int64_t F, int32_t k, int64_t num_nodes, BlockWs* w) {
    const int64_t f = F > 0 ? F : 1;
    const int64_t ecap = f * k;
    const int64_t nwords = (num_nodes + 31) / 32 > 0 ? (num_nodes + 31) / 32 : 1;
    const int64_t W = (f + 15) / 16;
    w->cnt = cv.template take<int32_t>(f + 1);
    w->off = cv.template take<int64_t>(f + 2);
    w->err = cv.template take<int32_t>(64);
    w->edge_dst = cv.template take<int32_t>(ecap);
    w->edge_src = cv.template take<int64_t>(ecap);
    w->edge_val = cv.template take<float>(ecap);
    w->src_local = cv.template take<int32_t>(ecap);
    w->wcnt = cv.template take<int32_t>(nwords);
    w->wprefix = cv.template take<int64_t>(nwords + 1);
    w->wtiles = cv.template take<int32_t>(W + 1);
    int64_t m = f > nwords ? f : nwords;
    w->scan_bytes = scan_workspace_bytes(m);
    w->scan_ws = cv.template take<char>(w->scan_bytes);
}

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


// ---------------------------------------------------------------------------
// fused hop: sample + relabel + BCSR block, one synchronisation
// ---------------------------------------------------------------------------
extern "C" int grws_sample_state_init(int32_t* node_map, uint32_t* bitmap, int64_t num_nodes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(num_nodes >= 0, "sample_state_init: negative num_nodes");
    if (num_nodes == 0) return GRWS_OK;
    GRWS_CHECK_ARG(node_map && bitmap, "sample_state_init: null pointer");
    const int64_t nwords = (num_nodes + 31) / 32;
    int64_t blocks = (num_nodes + kBlk - 1) / kBlk;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fill_state_kernel, dim3((unsigned)blocks), dim3(kBlk), 0, stream, node_map, num_nodes, bitmap,
                       nwords);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

extern "C" size_t grws_sample_block_workspace_bytes(int64_t num_frontier, int32_t fanout, int64_t num_nodes) {
    if (num_frontier < 0 || fanout < 1 || fanout > kWave || num_nodes < 0) return 0;
    NullCarver nc;
    BlockWs w;
    carve_block(nc, num_frontier, fanout, num_nodes, &w);
    return nc.s.used + 256;
}

extern "C" int grws_sample_block_capacity(int64_t num_frontier, int32_t fanout, int32_t tile_cols, int64_t* max_src,
                                          int64_t* max_tiles) {
    clear_error();
    GRWS_CHECK_ARG(num_frontier >= 0, "sample_block_capacity: negative num_frontier");
    GRWS_CHECK_ARG(fanout >= 1 && fanout <= kWave, "sample_block_capacity: fanout must be in [1, 64]");
    GRWS_CHECK_ARG(tile_cols == 8 || tile_cols == 16, "sample_block_capacity: tile_cols must be 8 or 16");
    GRWS_CHECK_ARG(max_src && max_tiles, "sample_block_capacity: null output");
    const int64_t W = (num_frontier + 15) / 16;
    *max_src = num_frontier * (1 + (int64_t)fanout);
    *max_tiles = W * ((16 * (int64_t)fanout + tile_cols - 1) / tile_cols);
    return GRWS_OK;
}

extern "C" int grws_sample_block(const int64_t* indptr, const int32_t* indices, int64_t num_nodes, int64_t nnz,
                                 const int64_t* frontier, int64_t num_frontier, int32_t fanout, uint64_t seed,
                                 int32_t* node_map, uint32_t* bitmap, int32_t tile_cols, int32_t values_dtype,
                                 int64_t* next_frontier, int64_t max_src, int64_t* window_offset,
                                 int32_t* col_indices, void* values, int64_t max_tiles, void* workspace,
                                 size_t workspace_bytes, int64_t* counts_out, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    const int64_t F = num_frontier;
    GRWS_CHECK_ARG(num_nodes >= 0 && nnz >= 0 && F >= 0, "sample_block: negative size");
    GRWS_CHECK_ARG(fanout >= 1 && fanout <= kWave, "sample_block: fanout must be in [1, 64] (got %d)", fanout);
    GRWS_CHECK_ARG(tile_cols == 8 || tile_cols == 16, "sample_block: tile_cols must be 8 or 16");
    GRWS_CHECK_ARG(num_nodes <= INT32_MAX && F <= INT32_MAX, "sample_block: ids exceed int32 local ids");
    if (values_dtype != GRWS_F32 && values_dtype != GRWS_F16 && values_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "sample_block: unsupported values dtype %d", values_dtype);
    GRWS_CHECK_ARG(counts_out != nullptr && window_offset != nullptr, "sample_block: null output");
    int64_t cap_src = 0, cap_tiles = 0;
    GRWS_TRY(grws_sample_block_capacity(F, fanout, tile_cols, &cap_src, &cap_tiles));
    GRWS_CHECK_ARG(max_src >= cap_src && max_tiles >= cap_tiles,
                   "sample_block: outputs too small (src %lld < %lld or tiles %lld < %lld)", (long long)max_src,
                   (long long)cap_src, (long long)max_tiles, (long long)cap_tiles);
    counts_out[0] = counts_out[1] = counts_out[2] = 0;
    const int64_t W = (F + 15) / 16;
    if (F == 0) return fill_i64(window_offset, 1, 0, stream);
    GRWS_CHECK_ARG(indptr && frontier && node_map && bitmap && next_frontier && col_indices && values,
                   "sample_block: null pointer");
    if (nnz > 0) GRWS_CHECK_ARG(indices != nullptr, "sample_block: null indices");
    Carver cv(workspace, workspace_bytes);
    BlockWs w;
    carve_block(cv, F, fanout, num_nodes, &w);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "sample_block: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const int64_t nwords = (num_nodes + 31) / 32;

    GRWS_TRY(fill_i32(w.err, 1, 0, stream));
    // 1. sample (the kernels of grws_sample_hop)
    hipLaunchKernelGGL(hop_count_kernel, dim3(grid_for(F)), dim3(kBlk), 0, stream, indptr, nnz, num_nodes, frontier, F,
                       (int)fanout, w.cnt, w.err);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(w.cnt, w.off, F, false, w.scan_ws, w.scan_bytes, stream));
    hipLaunchKernelGGL(hop_sample_kernel, dim3(grid_for(F, kWavesPerBlock)), dim3(kBlk), 0, stream, indptr, indices,
                       nnz, num_nodes, frontier, F, (int)fanout, seed, w.off, w.edge_dst, w.edge_src, w.edge_val,
                       w.err);
    GRWS_LAUNCH_CHECK();
    // 2. relabel through the dense map and the new-source bitmap; the edge
    //    count is not known on the host, so edge kernels cover F * fanout
    //    slots and those past the count see edge_src = -1
    const int64_t ecap = F * (int64_t)fanout;
    hipLaunchKernelGGL(tail_fill_kernel, dim3(grid_for(ecap)), dim3(kBlk), 0, stream, w.off + F, w.edge_src, ecap);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(map_frontier_kernel, dim3(grid_for(F)), dim3(kBlk), 0, stream, frontier, F, num_nodes, node_map,
                       w.err);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(mark_new_kernel, dim3(grid_for(ecap)), dim3(kBlk), 0, stream, w.edge_src, ecap, num_nodes,
                       node_map, bitmap);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(word_popcount_kernel, dim3(grid_for(nwords)), dim3(kBlk), 0, stream, bitmap, nwords, w.wcnt);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(w.wcnt, w.wprefix, nwords, false, w.scan_ws, w.scan_bytes, stream));
    hipLaunchKernelGGL(copy_i64_kernel, dim3(grid_for(F)), dim3(kBlk), 0, stream, frontier, F, next_frontier);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(assign_local_kernel, dim3(grid_for(ecap)), dim3(kBlk), 0, stream, w.edge_src, ecap, num_nodes,
                       F, node_map, bitmap, w.wprefix, w.src_local, next_frontier);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(reset_state_kernel, dim3(grid_for(F > ecap ? F : ecap)), dim3(kBlk), 0, stream, frontier, F,
                       w.edge_src, ecap, num_nodes, node_map, bitmap);
    GRWS_LAUNCH_CHECK();
    // 3. per-window BCSR of the block (rows = frontier positions)
    const int vd = values_dtype;
#define GRWS_BLOCK_WINDOWS(FILL, VT)                                                                            \
    hipLaunchKernelGGL(block_window_kernel<VT>, dim3((unsigned)W), dim3(kBlk), 0, stream, FILL, w.off, F,          \
                       w.src_local, w.edge_val, (int)tile_cols, w.wtiles, window_offset, col_indices,             \
                       static_cast<VT*>(values))
    if (vd == GRWS_F32) GRWS_BLOCK_WINDOWS(0, float);
    else if (vd == GRWS_F16) GRWS_BLOCK_WINDOWS(0, _Float16);
    else GRWS_BLOCK_WINDOWS(0, __hip_bfloat16);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(w.wtiles, window_offset, W, false, w.scan_ws, w.scan_bytes, stream));
    if (vd == GRWS_F32) GRWS_BLOCK_WINDOWS(1, float);
    else if (vd == GRWS_F16) GRWS_BLOCK_WINDOWS(1, _Float16);
    else GRWS_BLOCK_WINDOWS(1, __hip_bfloat16);
#undef GRWS_BLOCK_WINDOWS
    GRWS_LAUNCH_CHECK();
    int64_t h[3] = {0, 0, 0};
    int32_t e = 0;
    GRWS_HIP(hipMemcpyAsync(&h[0], w.off + F, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&h[1], w.wprefix + nwords, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&h[2], window_offset + W, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&e, w.err, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    GRWS_TRY(report(e, "sample_block"));
    counts_out[0] = h[0];
    counts_out[1] = F + h[1];
    counts_out[2] = h[2];
    return GRWS_OK;
}
