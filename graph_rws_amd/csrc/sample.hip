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

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

enum : int32_t { kErrNode = 1, kErrIndptr = 2, kErrIndex = 4, kErrDup = 8, kErrDegree = 16, kErrCount = 32 };

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
    if (e & kErrCount) return set_error(GRWS_E_RANGE, "%s: the seed count in device memory is outside [0, max_seeds]", who);
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

// ---------------------------------------------------------------------------
// whole batch (grws_sample_blocks): every hop on the device, one sync
// ---------------------------------------------------------------------------
// Sizes stay on the device: each hop's frontier, edge and tile counts live in
// BatchCtr (in the caller's state buffer, all zero between calls), and every
// kernel is launched over the hop's host-side capacity, its surplus threads
// leaving at once.  Edges are stored in fixed slots: frontier node i owns
// slots [i k, i k + k), min(deg, k) of them filled in ascending CSR position
// and the rest -1, so no offset scan is needed.  The relabel ranks a new
// source by the count of new sources in earlier 1024-id groups (one scan
// over the group counts the marking kept) plus the set bits before it in its
// own group: work proportional to the batch and to num_nodes / 1024, not to
// the whole bitmap.
constexpr int kMaxHops = 8;
constexpr int kGroupShift = 10;  // 1024 ids (32 bitmap words) per group

constexpr int kESub = 16;   // sub-counters per hop's edge count (fewer atomics on one address)

struct BatchCtr {
    int64_t F[kMaxHops + 1];  // frontier size of each hop (F[h+1] = sources of hop h)
    int64_t E[kMaxHops];      // sampled edges of each hop
    int64_t Esub[kMaxHops][kESub];  // the count pass's per-window adds (window w into w % kESub)
    int64_t T[kMaxHops];      // tiles of each hop's block
    int64_t TT[kMaxHops];     // tiles of each hop's transposed block
    int32_t TM[kMaxHops];     // most tiles in one window of the transposed block
    int32_t err;
    uint32_t done;            // work-groups of the group scan that have finished
};
constexpr int64_t kCtrWords = (sizeof(BatchCtr) + 3) / 4;

inline int64_t bitmap_words(int64_t n) { return (n + 31) / 32; }
inline int64_t group_count(int64_t n) { return (n + (1 << kGroupShift) - 1) >> kGroupShift; }

// Frontier size of hop h: the seeds' count is F0, or with F0 < 0 (an
// enqueued batch, whose count lives in device memory) c->F[0].
__device__ __forceinline__ int64_t hop_frontier(const BatchCtr* c, int h, int64_t F0) {
    return h == 0 ? (F0 >= 0 ? F0 : c->F[0]) : c->F[h];
}

// An enqueued batch's seed count, read from device memory before hop 0.
__global__ void mh_start_kernel(const int64_t* __restrict__ num_seeds_dev, int64_t max_seeds,
                                BatchCtr* __restrict__ ctr) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const int64_t n = *num_seeds_dev;
    const bool ok = n >= 0 && n <= max_seeds;
    ctr->F[0] = ok ? n : 0;
    if (!ok) atomicOr(&ctr->err, kErrCount);
}

// The seeds' node map entries (hop 0's frontier positions), duplicates and
// bad ids flagged.  Later hops need no such pass: the node map keeps every
// entry through the batch (a hop's frontier is the previous frontier, at the
// same positions, followed by its new sources, which the count pass maps),
// and the last hop's fill pass clears it.
__global__ __launch_bounds__(kBlk) void mh_seed_kernel(const int64_t* __restrict__ indptr, int64_t nnz,
                                                       int64_t num_nodes, const int64_t* __restrict__ seeds,
                                                       int64_t F0, int32_t* __restrict__ node_map,
                                                       BatchCtr* __restrict__ ctr) {
    const int64_t F = hop_frontier(ctr, 0, F0);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0 && F0 >= 0) ctr->F[0] = F0;
    if (i >= F) return;
    const int64_t v = seeds[i];
    const NodeRange r = node_range(indptr, nnz, num_nodes, v);
    if (r.err) {
        atomicOr(&ctr->err, r.err);
    } else if (atomicExch(&node_map[v], (int32_t)i) != -1) {
        atomicOr(&ctr->err, kErrDup);
    }
}

// One wave per frontier node: the hop_sample_kernel draw into fixed slots,
// then the new sources' bits and group counts.
__global__ __launch_bounds__(kBlk) void mh_sample_kernel(const int64_t* __restrict__ indptr,
                                                         const int32_t* __restrict__ indices, int64_t nnz,
                                                         int64_t num_nodes, const int64_t* __restrict__ frontier,
                                                         int64_t F0, int h, int k, uint64_t seed,
                                                         const int32_t* __restrict__ node_map,
                                                         uint32_t* __restrict__ bitmap, int32_t* __restrict__ grpcnt,
                                                         int64_t* __restrict__ edge_src, float* __restrict__ edge_val,
                                                         BatchCtr* __restrict__ ctr) {
    const int64_t F = hop_frontier(ctr, h, F0);
    const int64_t i = (int64_t)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    if (i >= F) return;  // wave-uniform
    const int lane = lane_id();
    const int64_t v = frontier[i];
    const NodeRange r = node_range(indptr, nnz, num_nodes, v);
    if (r.err && lane == 0) atomicOr(&ctr->err, r.err);
    const int64_t deg = r.err ? 0 : r.deg;
    int64_t x = lane;
    int rank = lane;
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
        x = -1;
        for (int d = 0; d < k; ++d) {
            const int64_t td = readlane64(t, d);
            const bool taken = __ballot(lane < d && x == td) != 0ull;
            if (lane == d) x = taken ? j0 + d : td;
        }
        rank = 0;
        for (int e = 0; e < k; ++e) rank += readlane64(x, e) < x ? 1 : 0;
    }
    const int64_t slot0 = i * (int64_t)k;
    if (lane < n) {
        const int32_t s = indices[r.start + x];
        const int64_t o = slot0 + rank;
        edge_src[o] = (int64_t)s;
        float w = 0.0f;
        if (s >= 0 && (int64_t)s < num_nodes) {
            w = gcn_weight(deg, indptr[(int64_t)s + 1] - indptr[s]);
            if (node_map[s] < 0) {
                const uint32_t bit = 1u << (s & 31);
                if (!(atomicOr(&bitmap[s >> 5], bit) & bit)) atomicAdd(&grpcnt[s >> kGroupShift], 1);
            }
        } else {
            atomicOr(&ctr->err, kErrIndex);
        }
        edge_val[o] = w;
    } else if (lane < k) {
        edge_src[slot0 + lane] = -1;  // empty slot
    }
}

// Exclusive scan of the group counts: one work-group of 256 threads per
// slice of 1024 groups (lane t of the slice takes 4 consecutive counts)
// writes the in-slice prefixes and the slice total; the last work-group to
// finish (a ticket, no waiting) turns the slice totals into slice offsets and
// sets F[h+1] = F[h] + the number of new sources.
constexpr int kSliceGroups = 1024;
__global__ __launch_bounds__(kBlk) void mh_group_scan_kernel(const int32_t* __restrict__ grpcnt, int64_t ng,
                                                             int32_t* __restrict__ grpoff, int32_t* slicesum,
                                                             int32_t* __restrict__ sliceoff, int64_t nslices,
                                                             int64_t F0, int h, BatchCtr* __restrict__ ctr) {
    __shared__ int64_t tmp[kBlk / kWave + 1];
    __shared__ bool last;
    const int64_t base = (int64_t)blockIdx.x * kSliceGroups + 4 * threadIdx.x;
    int32_t v[4];
    int64_t t = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        v[q] = base + q < ng ? grpcnt[base + q] : 0;
        t += v[q];
    }
    int64_t total;
    const int64_t incl = block_incl_scan<kBlk>(t, tmp, &total);
    int64_t x = incl - t;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (base + q < ng) grpoff[base + q] = (int32_t)x;
        x += v[q];
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(&slicesum[blockIdx.x], (int32_t)total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __threadfence();
        last = atomicAdd(&ctr->done, 1u) == (uint32_t)(nslices - 1);
    }
    __syncthreads();
    if (!last) return;
    // every slice total is visible: exclusive scan of the nslices totals
    __threadfence();
    const int64_t per = (nslices + kBlk - 1) / kBlk;
    const int64_t b = threadIdx.x * per;
    const int64_t e = b + per < nslices ? b + per : nslices;
    int64_t sum = 0;
    for (int64_t k = b; k < e; ++k) sum += __hip_atomic_load(&slicesum[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int64_t inc2 = block_incl_scan<kBlk>(sum, tmp, &total);
    int64_t run = inc2 - sum;
    for (int64_t k = b; k < e; ++k) {
        sliceoff[k] = (int32_t)run;
        run += __hip_atomic_load(&slicesum[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x == 0) {
        ctr->F[h + 1] = hop_frontier(ctr, h, F0) + total;
        ctr->done = 0u;
    }
}

// Local id of a slot's source s (edge_src[e]): -1 for an empty slot, 0 for
// an invalid id (the sampler flagged it), the frontier position of a
// frontier node, else F + the new sources of earlier groups + the set bits
// before it in its group (the group's 32 words are one 128-byte line); a new
// source also writes its global id at its place in the next frontier (every
// slot of that source writes the same value) and, with map_new (every hop but
// the last), its local id into the node map.
__device__ __forceinline__ int32_t mh_local_id(int64_t s, int64_t F, int64_t num_nodes,
                                               int32_t* __restrict__ node_map, bool map_new,
                                               const uint32_t* __restrict__ bitmap,
                                               const int32_t* __restrict__ grpoff,
                                               const int32_t* __restrict__ sliceoff,
                                               int64_t* __restrict__ next_frontier) {
    if (s < 0) return -1;
    if (s >= num_nodes) return 0;
    const int32_t l = node_map[s];
    if (l >= 0) return l;
    const int64_t g = s >> kGroupShift;
    const int wi = (int)((s >> 5) & 31);
    const u32x4_t* gw = reinterpret_cast<const u32x4_t*>(bitmap + (g << 5));
    int below = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const u32x4_t v = gw[q];
#pragma unroll
        for (int j = 0; j < 4; ++j) below += (4 * q + j < wi) ? __popc(v[j]) : 0;
    }
    below += __popc(bitmap[s >> 5] & ((1u << (s & 31)) - 1u));
    const int64_t local = F + sliceoff[g / kSliceGroups] + grpoff[g] + below;
    next_frontier[local] = s;
    // the next hop's frontier position of s; a slot of this hop that reads
    // the entry early takes the frontier branch above and gets the same id
    if (map_new) node_map[s] = (int32_t)local;
    return (int32_t)local;
}

// Count pass of a hop's block, one work-group per 16-row window, slots
// [16 w k, min(16 w + 16, F) k): the local id of every slot's source
// (mh_local_id) into src_local, the window's rows into the next frontier's
// first F entries, the window's tiles (its distinct local ids, counted by
// insertion into an LDS hash set: open addressing, at most half full; no
// sort, the fill pass sorts; over tc per tile) and its filled slots added to
// one of the hop's edge sub-counters.  The relabel state stays as it is here
// (other windows still read it); the fill pass restores it.
__global__ __launch_bounds__(kBlk) void mh_wcount_kernel(const int64_t* __restrict__ frontier, int64_t F0, int h,
                                                         int k, int64_t num_nodes,
                                                         const int64_t* __restrict__ edge_src,
                                                         int32_t* __restrict__ node_map, int map_new,
                                                         const uint32_t* __restrict__ bitmap,
                                                         const int32_t* __restrict__ grpoff,
                                                         const int32_t* __restrict__ sliceoff,
                                                         int32_t* __restrict__ src_local,
                                                         int64_t* __restrict__ next_frontier, int tc,
                                                         int32_t* __restrict__ wtiles,
                                                         BatchCtr* __restrict__ ctr) {
    __shared__ uint32_t tab[2 * kWinEdges];
    __shared__ int64_t scan_tmp[kBlk / kWave + 1];
    const int tid = threadIdx.x;
    const int64_t F = hop_frontier(ctr, h, F0);
    const int64_t W = (F + 15) / 16;
    const int64_t w = blockIdx.x;
    if (w >= W) {
        if (tid == 0) wtiles[w] = 0;
        return;
    }
    const int64_t r0 = w * 16;
    const int rows = (int)(F - r0 < 16 ? F - r0 : 16);
    const int64_t s0 = r0 * k;
    const int ns = rows * k;  // <= kWinEdges
    int TS = 64;
    while (TS < 2 * ns) TS <<= 1;
    if (tid < rows) next_frontier[r0 + tid] = frontier[r0 + tid];
    for (int i = tid; i < TS; i += kBlk) tab[i] = 0xffffffffu;
    __syncthreads();
    // distinct ids (low 32 bits) and filled slots (high 32 bits) in one sum
    int64_t cnt = 0;
    for (int i = tid; i < ns; i += kBlk) {
        const int32_t c = mh_local_id(edge_src[s0 + i], F, num_nodes, node_map, map_new != 0, bitmap, grpoff,
                                      sliceoff, next_frontier);
        src_local[s0 + i] = c;
        if (c < 0) continue;
        cnt += (int64_t)1 << 32;
        uint32_t q = ((uint32_t)c * 0x9E3779B1u) >> 16;
        for (;;) {  // at most TS probes: the set holds at most ns < TS ids
            q &= (uint32_t)(TS - 1);
            const uint32_t old = atomicCAS(&tab[q], 0xffffffffu, (uint32_t)c);
            if (old == 0xffffffffu) {
                ++cnt;
                break;
            }
            if (old == (uint32_t)c) break;
            ++q;
        }
    }
    int64_t total;
    block_incl_scan<kBlk>(cnt, scan_tmp, &total);
    if (tid == 0) {
        const int64_t distinct = total & 0xffffffffll;
        wtiles[w] = (int32_t)((distinct + tc - 1) / tc);
        if (total >> 32)  // sampled edges, spread over the hop's sub-counters
            atomicAdd((unsigned long long*)&ctr->Esub[h][w % kESub], (unsigned long long)(total >> 32));
    }
}

// Fill pass of a hop's block, one work-group per 16-row window, slots
// [16 w k, min(16 w + 16, F) k): sorted in LDS by (column, row, slot), the
// distinct columns numbered and the window's tiles written, at the offset
// the count pass's tiles of the earlier windows sum to; then the window's share of the
// relabel state restored (its sources' bitmap words and group counts, and in
// the last hop its rows' node map entries; every local id is known by now).  Same rules as
// block_window_kernel (the last of duplicate (row, column) slots wins).
template <typename VT>
__global__ __launch_bounds__(256) void mh_window_kernel(const int64_t* __restrict__ frontier, int64_t F0,
                                                        int h, int k, const int32_t* __restrict__ src_local,
                                                        const int64_t* __restrict__ edge_src,
                                                        const float* __restrict__ edge_val, int tc,
                                                        const int32_t* __restrict__ wtiles,
                                                        int64_t* __restrict__ window_offset,
                                                        int32_t* __restrict__ out_cols, VT* __restrict__ out_vals,
                                                        int64_t num_nodes, int32_t* __restrict__ node_map,
                                                        int last, uint32_t* __restrict__ bitmap,
                                                        int32_t* __restrict__ grpcnt, BatchCtr* __restrict__ ctr) {
    __shared__ uint64_t key[kWinEdges];
    __shared__ int32_t pos[kWinEdges];
    __shared__ int64_t scan_tmp[kBlk / kWave + 1];
    const int tid = threadIdx.x;
    const int64_t F = hop_frontier(ctr, h, F0);
    const int64_t W = (F + 15) / 16;
    const int64_t w = blockIdx.x;
    if (w == 0 && tid == 0) window_offset[0] = 0;
    if (w >= W) return;
    const int64_t r0 = w * 16;
    const int rows = (int)(F - r0 < 16 ? F - r0 : 16);
    const int64_t s0 = r0 * k;
    const int ns = rows * k;  // <= kWinEdges
    int P = 1;
    while (P < ns) P <<= 1;
    for (int i = tid; i < P; i += kBlk) {
        uint64_t kk = ~0ull;
        if (i < ns) {
            const int32_t c = src_local[s0 + i];
            if (c >= 0) kk = ((uint64_t)(uint32_t)c << 14) | ((uint64_t)(i / k) << 10) | (uint64_t)i;
        }
        key[i] = kk;
    }
    // restore the state this hop changed: bitmap words and group counts of
    // its sources (the count pass, which read them, has finished); in the
    // last hop also the node map of the window's rows, which by then are
    // every node the batch mapped
    if (last && tid < rows) {
        const int64_t v = frontier[r0 + tid];
        if (v >= 0 && v < num_nodes) node_map[v] = -1;
    }
    for (int i = tid; i < ns; i += kBlk) {
        const int64_t s = edge_src[s0 + i];
        if (s >= 0 && s < num_nodes) {
            bitmap[s >> 5] = 0u;
            grpcnt[s >> kGroupShift] = 0;
        }
    }
    __syncthreads();
    if (P <= 128) {
        // up to 128 slots (fanout <= 8): each key's place is the number of
        // keys before it (keys are distinct but for the ~0 padding, whose
        // ties go by position): one pass over LDS and two barriers instead
        // of the 28 barrier-separated steps of a bitonic network (measured
        // 9.8 -> 8.3 us per c5 hop of fanout 5; at 256 slots the quadratic
        // pass is the slower one)
        const uint64_t mine = tid < P ? key[tid] : 0ull;
        int rank = 0;
        if (tid < P) {
#pragma unroll 8
            for (int q = 0; q < P; ++q) {
                const uint64_t o = key[q];
                rank += (o < mine || (o == mine && q < tid)) ? 1 : 0;
            }
        }
        __syncthreads();
        if (tid < P) key[rank] = mine;
        __syncthreads();
    } else {
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
    }
    int flags = 0, cnt = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = tid * 4 + q;
        const bool f = i < P && key[i] != ~0ull && (i == 0 || (key[i] >> 14) != (key[i - 1] >> 14));
        flags |= (f ? 1 : 0) << q;
        cnt += f ? 1 : 0;
    }
    int64_t total;
    const int64_t incl = block_incl_scan<kBlk>(cnt, scan_tmp, &total);
    int run = (int)(incl - cnt);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = tid * 4 + q;
        if (i < P) {
            run += (flags >> q) & 1;
            pos[i] = run - 1;
        }
    }
    const int64_t tiles = (total + tc - 1) / tc;
    // the window's first tile: the count pass's tiles of the windows before
    // it, summed by this work-group (no scan launch; at most a few thousand
    // windows per hop); the last window writes the total
    int64_t part = 0;
    for (int64_t v = tid; v < w; v += kBlk) part += wtiles[v];
    int64_t wo;
    block_incl_scan<kBlk>(part, scan_tmp, &wo);
    if (tid == 0) {
        window_offset[w + 1] = wo + tiles;
        if (w == W - 1) ctr->T[h] = wo + tiles;
    }
    for (int64_t i = tid; i < tiles * tc; i += kBlk) out_cols[wo * tc + i] = -1;
    for (int64_t i = tid; i < tiles * 16 * tc; i += kBlk) out_vals[wo * 16 * tc + i] = cvt_value<VT>(0.0f);
    __syncthreads();
    for (int i = tid; i < P; i += kBlk) {
        const uint64_t kk = key[i];
        if (kk == ~0ull) continue;
        const int p = pos[i];
        const int64_t tile = wo + p / tc;
        const int c = p % tc;
        if (i == 0 || (key[i - 1] >> 14) != (kk >> 14)) out_cols[tile * tc + c] = (int32_t)(kk >> 14);
        if (i + 1 >= P || (key[i + 1] >> 10) != (kk >> 10)) {
            const int r = (int)((kk >> 10) & 15u);
            out_vals[(tile * 16 + r) * tc + c] = cvt_value<VT>(edge_val[s0 + (int64_t)(kk & 1023u)]);
        }
    }
}

// --- transposed blocks -----------------------------------------------------
// A^T of hop h's block: windows of 16 sources, columns = the hop's frontier
// rows, the BCSR that a build of the block's transpose makes (every cell of
// the block with a nonzero value, in a window's distinct rows ascending).
// Built from the hop's slots without a host sync: a stable radix sort by
// source window keeps slot order inside a window, so a window's slots come
// out ordered by frontier row (slot / k) and, within a row, by slot.

__device__ __forceinline__ bool value_nonzero(float v) { return v != 0.0f; }
__device__ __forceinline__ bool value_nonzero(_Float16 v) { return (float)v != 0.0f; }
__device__ __forceinline__ bool value_nonzero(__hip_bfloat16 v) { return __bfloat162float(v) != 0.0f; }

// Key of every slot: its source's window, or wcap (after every window) for an
// empty slot, a slot past the hop's edges, or a value that is zero in VT.
template <typename VT>
__global__ __launch_bounds__(kBlk) void mh_tkeys_kernel(int64_t F0, int h, int k, const int32_t* __restrict__ src_local,
                                                        const float* __restrict__ edge_val, int64_t ecap, int64_t wcap,
                                                        uint64_t* __restrict__ keys, uint32_t* __restrict__ pay,
                                                        const BatchCtr* __restrict__ ctr) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= ecap) return;
    const int64_t F = hop_frontier(ctr, h, F0);
    uint64_t kk = (uint64_t)wcap;
    if (e < F * (int64_t)k) {
        const int32_t c = src_local[e];
        if (c >= 0 && value_nonzero(cvt_value<VT>(edge_val[e]))) kk = (uint64_t)(c >> 4);
    }
    keys[e] = kk;
    pay[e] = (uint32_t)e;
}

// First slot of every transposed window in the sorted keys: tstart[w] = the
// first position whose key is >= w, for the windows that hold the hop's
// sources, w = 0 .. Wa = ceil(sources / 16) (valid keys lie below Wa, the
// empty-slot key wcap after them).  Position i starts the windows
// (key[i-1], key[i]], position ecap those after the last key, both clamped
// to Wa, so each entry is written once and no thread walks the capacity's
// unused windows; the windows' kernels then read their ranges instead of
// searching for them.
__global__ __launch_bounds__(kBlk) void mh_tbounds_kernel(int h, const uint64_t* __restrict__ keys, int64_t ecap,
                                                          int64_t wcap, int64_t* __restrict__ tstart,
                                                          const BatchCtr* __restrict__ ctr) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i > ecap) return;
    const int64_t Wa = (ctr->F[h + 1] + 15) / 16;
    const int64_t lo = i == 0 ? -1 : (int64_t)keys[i - 1];
    int64_t hi = i == ecap ? wcap + 1 : (int64_t)keys[i];
    if (hi > Wa) hi = Wa;
    for (int64_t w = lo + 1; w <= hi; ++w) tstart[w] = i;
}

// Per transposed window: its distinct frontier rows -> tiles.  One wave per
// window (a window holds a few dozen slots: ballots count them, no barriers),
// waves striding over the capacity's windows.
__global__ __launch_bounds__(kBlk) void mh_tcount_kernel(int h, int k, const int64_t* __restrict__ tstart,
                                                         const uint32_t* __restrict__ pay, int tc, int64_t wcap,
                                                         int32_t* __restrict__ wtiles, BatchCtr* __restrict__ ctr) {
    __shared__ int32_t wmax[kBlk / kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t nwaves = (int64_t)gridDim.x * (kBlk / kWave);
    const int64_t Wa = (ctr->F[h + 1] + 15) / 16;
    int32_t most = 0;
    for (int64_t w = ((int64_t)blockIdx.x * kBlk + threadIdx.x) / kWave; w < wcap; w += nwaves) {  // uniform per wave
        if (w >= Wa) {  // past the hop's sources: no slots
            if (lane == 0) wtiles[w] = 0;
            continue;
        }
        const int64_t lo = tstart[w];
        const int64_t hi = tstart[w + 1];
        int64_t distinct = 0;
        for (int64_t b = lo; b < hi; b += kWave) {
            const int64_t i = b + lane;
            const bool f = i < hi && (i == lo || pay[i - 1] / (uint32_t)k != pay[i] / (uint32_t)k);
            distinct += __popcll(__ballot(f));
        }
        const int32_t t = (int32_t)((distinct + tc - 1) / tc);
        if (lane == 0) wtiles[w] = t;
        most = t > most ? t : most;
    }
    // one atomic per work-group: thousands of windows updating one counter
    // would serialise at the L2
    if (lane == 0) wmax[threadIdx.x / kWave] = most;
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t m = 0;
#pragma unroll
        for (int i = 0; i < kBlk / kWave; ++i) m = wmax[i] > m ? wmax[i] : m;
        if (m > 0) atomicMax(&ctr->TM[h], m);
    }
}

// One work-group per transposed window: column = frontier row, value at the
// source's row of the window; of slots repeating a (row, source) pair the
// last one's value is stored, as in the block.  (A wave per window measured
// slower here: the window's chain of dependent loads then ran on one wave
// per SIMD slot instead of four.)
template <typename VT>
__global__ __launch_bounds__(kBlk) void mh_tfill_kernel(int h, int k, const int64_t* __restrict__ tstart,
                                                        const uint32_t* __restrict__ pay, int64_t wcap,
                                                        int tc, const int32_t* __restrict__ src_local,
                                                        const float* __restrict__ edge_val,
                                                        const int64_t* __restrict__ t_win, int32_t* __restrict__ out_cols,
                                                        void* __restrict__ out_vals_, BatchCtr* __restrict__ ctr) {
    __shared__ int64_t tmp[kBlk / kWave + 1];
    VT* __restrict__ out_vals = static_cast<VT*>(out_vals_);
    const int tid = threadIdx.x;
    const int64_t w = blockIdx.x;
    if (w == 0 && tid == 0) ctr->TT[h] = t_win[wcap];
    const int64_t wo = t_win[w];
    const int64_t tiles = t_win[w + 1] - wo;
    if (tiles <= 0) return;  // uniform over the work-group
    for (int64_t i = tid; i < tiles * tc; i += kBlk) out_cols[wo * tc + i] = -1;
    for (int64_t i = tid; i < tiles * 16 * tc; i += kBlk) out_vals[wo * 16 * tc + i] = cvt_value<VT>(0.0f);
    __syncthreads();
    const int64_t lo = tstart[w];
    const int64_t hi = tstart[w + 1];
    int64_t run = 0;
    for (int64_t b = lo; b < hi; b += kBlk) {  // uniform over the work-group
        const int64_t i = b + tid;
        const bool v = i < hi;
        uint32_t e = 0, d = 0;
        int f = 0;
        if (v) {
            e = pay[i];
            d = e / (uint32_t)k;
            f = (i == lo || pay[i - 1] / (uint32_t)k != d) ? 1 : 0;
        }
        int64_t tot;
        const int64_t inc = block_incl_scan<kBlk>(f, tmp, &tot);
        if (v) {
            const int64_t p = run + inc - 1;  // the row's position among the window's distinct rows
            const int64_t tile = wo + p / tc;
            const int col = (int)(p % tc);
            if (f) out_cols[tile * tc + col] = (int32_t)d;
            const int32_t c = src_local[e];
            bool last = true;
            for (int64_t j = i + 1; j < hi; ++j) {  // the row's later slots in this window (at most k)
                const uint32_t ej = pay[j];
                if (ej / (uint32_t)k != d) break;
                if (src_local[ej] == c) {
                    last = false;
                    break;
                }
            }
            if (last) out_vals[(tile * 16 + (c & 15)) * tc + col] = cvt_value<VT>(edge_val[e]);
        }
        run += tot;
    }
}

// Copies the batch counters out and clears them for the next call:
// out = F[0..H], E[H], T[H], TT[H], TM[H], err.
__global__ void mh_finish_kernel(BatchCtr* __restrict__ ctr, int64_t* __restrict__ out, int H) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    for (int h = 0; h <= H; ++h) out[h] = ctr->F[h];
    for (int h = 0; h < H; ++h) {
        int64_t e = ctr->E[h];
#pragma unroll
        for (int j = 0; j < kESub; ++j) e += ctr->Esub[h][j];
        out[H + 1 + h] = e;
        out[2 * H + 1 + h] = ctr->T[h];
        out[3 * H + 1 + h] = ctr->TT[h];
        out[4 * H + 1 + h] = ctr->TM[h];
    }
    out[5 * H + 1] = ctr->err;
    for (int h = 0; h <= kMaxHops; ++h) ctr->F[h] = 0;
    for (int h = 0; h < kMaxHops; ++h) {
        ctr->E[h] = ctr->T[h] = ctr->TT[h] = 0;
        for (int j = 0; j < kESub; ++j) ctr->Esub[h][j] = 0;
        ctr->TM[h] = 0;
    }
    ctr->err = 0;
}

// Host-side capacities of a batch: frontier, edge slots, windows and tiles
// of each hop.
struct HopCaps {
    int64_t F[kMaxHops + 1], E[kMaxHops], W[kMaxHops], T[kMaxHops];
    int64_t WT[kMaxHops], TT[kMaxHops];  // transposed block: windows, tiles
};

HopCaps hop_caps(int64_t num_seeds, const int32_t* fanouts, int H, int tc, int64_t num_nodes) {
    HopCaps c{};
    c.F[0] = num_seeds;
    for (int h = 0; h < H; ++h) {
        const int64_t k = fanouts[h];
        c.E[h] = c.F[h] * k;
        c.W[h] = (c.F[h] + 15) / 16;
        c.T[h] = c.W[h] * ((16 * k + tc - 1) / tc);
        // the next frontier is this one plus at most min(edges, num_nodes)
        // new sources
        const int64_t nf = c.F[h] * (1 + k);
        const int64_t lim = c.F[h] + num_nodes;
        c.F[h + 1] = nf < lim ? nf : lim;
        // windows of 16 sources; a window's tiles are at most one partial
        // tile more than its edges fill
        c.WT[h] = (c.F[h + 1] + 15) / 16;
        c.TT[h] = c.WT[h] + (c.E[h] + tc - 1) / tc;
    }
    return c;
}

struct BatchWs {
    int64_t* edge_src;
    float* edge_val;
    int32_t* src_local;
    int32_t* grpoff;
    int32_t* slicesum;
    int32_t* sliceoff;
    int32_t* wtiles;
    int64_t* out;
    char* scan_ws;
    size_t scan_bytes;
    // transposed blocks (carved only when a hop asks for one)
    uint64_t *tka, *tkb;
    uint32_t *tpa, *tpb;
    int64_t* tstart;
    char* sort_ws;
    size_t sort_bytes;
};

template <typename C>
void carve_batch(C& cv, const HopCaps& c, int H, int64_t num_nodes, const int32_t* thops, BatchWs* w) {
    int64_t emax = 1, wmax = 1, etmax = 0;
    for (int h = 0; h < H; ++h) {
        emax = c.E[h] > emax ? c.E[h] : emax;
        wmax = c.W[h] > wmax ? c.W[h] : wmax;
        if (thops && thops[h]) {
            etmax = c.E[h] > etmax ? c.E[h] : etmax;
            wmax = c.WT[h] > wmax ? c.WT[h] : wmax;
        }
    }
    w->edge_src = cv.template take<int64_t>(emax);
    w->edge_val = cv.template take<float>(emax);
    w->src_local = cv.template take<int32_t>(emax);
    w->grpoff = cv.template take<int32_t>(group_count(num_nodes) + 1);
    w->slicesum = cv.template take<int32_t>(group_count(num_nodes) / kSliceGroups + 2);
    w->sliceoff = cv.template take<int32_t>(group_count(num_nodes) / kSliceGroups + 2);
    w->wtiles = cv.template take<int32_t>(wmax + 1);
    w->out = cv.template take<int64_t>(5 * kMaxHops + 4);
    w->scan_bytes = scan_workspace_bytes(wmax);
    w->scan_ws = cv.template take<char>(w->scan_bytes);
    w->tka = w->tkb = nullptr;
    w->tpa = w->tpb = nullptr;
    w->tstart = nullptr;
    w->sort_ws = nullptr;
    w->sort_bytes = 0;
    if (etmax > 0) {
        w->tka = cv.template take<uint64_t>(etmax);
        w->tkb = cv.template take<uint64_t>(etmax);
        w->tpa = cv.template take<uint32_t>(etmax);
        w->tpb = cv.template take<uint32_t>(etmax);
        w->tstart = cv.template take<int64_t>(wmax + 2);
        w->sort_bytes = radix_sort_workspace_bytes(etmax);
        w->sort_ws = cv.template take<char>(w->sort_bytes);
    }
}

// State buffer of grws_sample_blocks (uint32 words): the new-source bitmap
// (padded to whole groups), the group counts, then BatchCtr on an 8-byte
// boundary.  Its first ceil(num_nodes / 32) words are the bitmap that
// grws_sample_block and grws_repack_* use.
struct StateLayout {
    int64_t groups, grp_off, ctr_off, words;
};

StateLayout state_layout(int64_t num_nodes) {
    StateLayout l;
    l.groups = group_count(num_nodes > 0 ? num_nodes : 1);
    l.grp_off = l.groups * 32;
    l.ctr_off = (l.grp_off + l.groups + 1) & ~(int64_t)1;
    l.words = l.ctr_off + kCtrWords;
    return l;
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

// ---------------------------------------------------------------------------
// whole batch: every hop, one synchronisation
// ---------------------------------------------------------------------------
extern "C" size_t grws_sample_blocks_state_words(int64_t num_nodes) {
    if (num_nodes < 0) return 0;
    return (size_t)state_layout(num_nodes).words;
}

extern "C" int grws_sample_blocks_state_init(int32_t* node_map, uint32_t* state, int64_t num_nodes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(num_nodes >= 0, "sample_blocks_state_init: negative num_nodes");
    GRWS_CHECK_ARG(state != nullptr && (node_map != nullptr || num_nodes == 0),
                   "sample_blocks_state_init: null pointer");
    GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(state) % 16 == 0, "sample_blocks_state_init: state not 16-byte aligned");
    const StateLayout l = state_layout(num_nodes);
    int64_t blocks = ((num_nodes > l.words ? num_nodes : l.words) + kBlk - 1) / kBlk;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(fill_state_kernel, dim3((unsigned)blocks), dim3(kBlk), 0, stream, node_map, num_nodes, state,
                       l.words);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

extern "C" int grws_sample_blocks_capacity(int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                                           int32_t tile_cols, int64_t num_nodes, int64_t* max_src,
                                           int64_t* max_tiles) {
    clear_error();
    GRWS_CHECK_ARG(num_seeds >= 0 && num_nodes >= 0, "sample_blocks_capacity: negative size");
    GRWS_CHECK_ARG(num_hops >= 1 && num_hops <= kMaxHops, "sample_blocks_capacity: num_hops must be in [1, %d]",
                   kMaxHops);
    GRWS_CHECK_ARG(fanouts && max_src && max_tiles, "sample_blocks_capacity: null pointer");
    GRWS_CHECK_ARG(tile_cols == 8 || tile_cols == 16, "sample_blocks_capacity: tile_cols must be 8 or 16");
    for (int h = 0; h < num_hops; ++h)
        GRWS_CHECK_ARG(fanouts[h] >= 1 && fanouts[h] <= kWave, "sample_blocks_capacity: fanout %d outside [1, 64]",
                       fanouts[h]);
    const HopCaps c = hop_caps(num_seeds, fanouts, num_hops, tile_cols, num_nodes);
    for (int h = 0; h < num_hops; ++h) {
        max_src[h] = c.F[h + 1];
        max_tiles[h] = c.T[h];
    }
    return GRWS_OK;
}

static size_t blocks_workspace_bytes(int64_t num_seeds, const int32_t* fanouts, int32_t num_hops, int32_t tile_cols,
                                     int64_t num_nodes, const int32_t* thops) {
    if (num_seeds < 0 || num_nodes < 0 || !fanouts || num_hops < 1 || num_hops > kMaxHops) return 0;
    for (int h = 0; h < num_hops; ++h)
        if (fanouts[h] < 1 || fanouts[h] > kWave) return 0;
    const HopCaps c = hop_caps(num_seeds, fanouts, num_hops, tile_cols == 8 ? 8 : 16, num_nodes);
    NullCarver nc;
    BatchWs w;
    carve_batch(nc, c, num_hops, num_nodes, thops, &w);
    return nc.s.used + 256;
}

extern "C" size_t grws_sample_blocks_workspace_bytes(int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                                                     int32_t tile_cols, int64_t num_nodes) {
    return blocks_workspace_bytes(num_seeds, fanouts, num_hops, tile_cols, num_nodes, nullptr);
}

extern "C" size_t grws_sample_blocks_transposed_workspace_bytes(int64_t num_seeds, const int32_t* fanouts,
                                                                int32_t num_hops, int32_t tile_cols, int64_t num_nodes,
                                                                const int32_t* transpose_hops) {
    return blocks_workspace_bytes(num_seeds, fanouts, num_hops, tile_cols, num_nodes, transpose_hops);
}

extern "C" int grws_sample_blocks_transposed_capacity(int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                                                      int32_t tile_cols, int64_t num_nodes, int64_t* max_t_windows,
                                                      int64_t* max_t_tiles) {
    clear_error();
    GRWS_CHECK_ARG(num_seeds >= 0 && num_nodes >= 0, "sample_blocks_transposed_capacity: negative size");
    GRWS_CHECK_ARG(num_hops >= 1 && num_hops <= kMaxHops,
                   "sample_blocks_transposed_capacity: num_hops must be in [1, %d]", kMaxHops);
    GRWS_CHECK_ARG(fanouts && max_t_windows && max_t_tiles, "sample_blocks_transposed_capacity: null pointer");
    GRWS_CHECK_ARG(tile_cols == 8 || tile_cols == 16, "sample_blocks_transposed_capacity: tile_cols must be 8 or 16");
    for (int h = 0; h < num_hops; ++h)
        GRWS_CHECK_ARG(fanouts[h] >= 1 && fanouts[h] <= kWave,
                       "sample_blocks_transposed_capacity: fanout %d outside [1, 64]", fanouts[h]);
    const HopCaps c = hop_caps(num_seeds, fanouts, num_hops, tile_cols, num_nodes);
    for (int h = 0; h < num_hops; ++h) {
        max_t_windows[h] = c.WT[h];
        max_t_tiles[h] = c.TT[h];
    }
    return GRWS_OK;
}

static int sample_blocks_impl(const int64_t* indptr, const int32_t* indices, int64_t num_nodes, int64_t nnz,
                              const int64_t* seeds, int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                              uint64_t seed, int32_t* node_map, uint32_t* state, int32_t tile_cols,
                              int32_t values_dtype, int64_t* const* next_frontier, int64_t* const* window_offset,
                              int32_t* const* col_indices, void* const* values, const int32_t* thops,
                              int64_t* const* t_window_offset, int32_t* const* t_col_indices, void* const* t_values,
                              void* workspace, size_t workspace_bytes, int64_t* counts_out, int per_hop,
                              const int64_t* num_seeds_dev, int64_t* counts_dev, hipStream_t stream) {
    const int H = num_hops;
    GRWS_CHECK_ARG(num_nodes >= 0 && nnz >= 0 && num_seeds >= 0, "sample_blocks: negative size");
    GRWS_CHECK_ARG(num_nodes <= INT32_MAX, "sample_blocks: ids exceed int32 local ids");
    GRWS_CHECK_ARG(H >= 1 && H <= kMaxHops, "sample_blocks: num_hops must be in [1, %d]", kMaxHops);
    GRWS_CHECK_ARG(fanouts && (counts_out || counts_dev), "sample_blocks: null pointer");
    GRWS_CHECK_ARG(tile_cols == 8 || tile_cols == 16, "sample_blocks: tile_cols must be 8 or 16");
    if (values_dtype != GRWS_F32 && values_dtype != GRWS_F16 && values_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "sample_blocks: unsupported values dtype %d", values_dtype);
    for (int h = 0; h < H; ++h)
        GRWS_CHECK_ARG(fanouts[h] >= 1 && fanouts[h] <= kWave, "sample_blocks: fanout %d outside [1, 64]", fanouts[h]);
    const HopCaps c = hop_caps(num_seeds, fanouts, H, tile_cols, num_nodes);
    GRWS_CHECK_ARG(c.F[H] <= INT32_MAX, "sample_blocks: a hop could exceed int32 local ids");
    if (counts_out)
        for (int h = 0; h < per_hop * H; ++h) counts_out[h] = 0;
    bool any_t = false;
    for (int h = 0; h < H; ++h) any_t = any_t || (thops && thops[h]);
    if (any_t) {
        GRWS_CHECK_ARG(t_window_offset && t_col_indices && t_values, "sample_blocks: null transposed outputs");
        for (int h = 0; h < H; ++h)
            if (thops[h]) {
                GRWS_CHECK_ARG(t_window_offset[h] && t_col_indices[h] && t_values[h],
                               "sample_blocks: null transposed output of hop %d", h);
                GRWS_CHECK_ARG(c.E[h] <= (int64_t)UINT32_MAX, "sample_blocks: hop %d has too many edge slots", h);
            }
    }
    if (num_seeds == 0 && !num_seeds_dev) {
        for (int h = 0; h < H; ++h) GRWS_TRY(fill_i64(window_offset[h], 1, 0, stream));
        for (int h = 0; h < H; ++h)
            if (any_t && thops[h]) GRWS_TRY(fill_i64(t_window_offset[h], 1, 0, stream));
        return GRWS_OK;
    }
    GRWS_CHECK_ARG(indptr && seeds && node_map && state && next_frontier && window_offset && col_indices && values,
                   "sample_blocks: null pointer");
    for (int h = 0; h < H; ++h)
        GRWS_CHECK_ARG(next_frontier[h] && window_offset[h] && col_indices[h] && values[h],
                       "sample_blocks: null output of hop %d", h);
    if (nnz > 0) GRWS_CHECK_ARG(indices != nullptr, "sample_blocks: null indices");
    GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(state) % 16 == 0, "sample_blocks: state not 16-byte aligned");
    Carver cv(workspace, workspace_bytes);
    BatchWs w;
    carve_batch(cv, c, H, num_nodes, any_t ? thops : nullptr, &w);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "sample_blocks: workspace too small (%zu < %zu)", workspace_bytes,
                                 cv.used);
    const StateLayout l = state_layout(num_nodes);
    uint32_t* bitmap = state;
    int32_t* grpcnt = reinterpret_cast<int32_t*>(state + l.grp_off);
    BatchCtr* ctr = reinterpret_cast<BatchCtr*>(state + l.ctr_off);
    const int tc = tile_cols;
    // kernels take the seed count as an argument, or read it from the
    // counters (-1) when it lives in device memory
    const int64_t F0 = num_seeds_dev ? -1 : num_seeds;
    if (num_seeds_dev) {
        hipLaunchKernelGGL(mh_start_kernel, dim3(1), dim3(64), 0, stream, num_seeds_dev, num_seeds, ctr);
        GRWS_LAUNCH_CHECK();
    }
    for (int h = 0; h < H; ++h) {
        const int k = fanouts[h];
        const int64_t Fc = c.F[h], Wc = c.W[h];
        const int64_t* fr = h == 0 ? seeds : next_frontier[h - 1];
        if (h == 0) {
            hipLaunchKernelGGL(mh_seed_kernel, dim3(grid_for(Fc)), dim3(kBlk), 0, stream, indptr, nnz, num_nodes,
                               fr, F0, node_map, ctr);
            GRWS_LAUNCH_CHECK();
        }
        hipLaunchKernelGGL(mh_sample_kernel, dim3(grid_for(Fc, kWavesPerBlock)), dim3(kBlk), 0, stream, indptr,
                           indices, nnz, num_nodes, fr, F0, h, k, seed, node_map, bitmap, grpcnt, w.edge_src,
                           w.edge_val, ctr);
        GRWS_LAUNCH_CHECK();
        const int64_t nslices = (l.groups + kSliceGroups - 1) / kSliceGroups;
        hipLaunchKernelGGL(mh_group_scan_kernel, dim3((unsigned)nslices), dim3(kBlk), 0, stream, grpcnt, l.groups,
                           w.grpoff, w.slicesum, w.sliceoff, nslices, F0, h, ctr);
        GRWS_LAUNCH_CHECK();
        hipLaunchKernelGGL(mh_wcount_kernel, dim3((unsigned)Wc), dim3(kBlk), 0, stream, fr, F0, h, k, num_nodes,
                           w.edge_src, node_map, (int)(h + 1 < H), bitmap, w.grpoff, w.sliceoff, w.src_local,
                           next_frontier[h], tc, w.wtiles, ctr);
        GRWS_LAUNCH_CHECK();
#define GRWS_MH_WINDOWS(VT)                                                                                        \
    hipLaunchKernelGGL(mh_window_kernel<VT>, dim3((unsigned)Wc), dim3(kBlk), 0, stream, fr, F0, h, k, w.src_local,   \
                       w.edge_src, w.edge_val, tc, w.wtiles, window_offset[h], col_indices[h],                        \
                       static_cast<VT*>(values[h]), num_nodes, node_map, (int)(h + 1 == H), bitmap, grpcnt, ctr)
        if (values_dtype == GRWS_F32) GRWS_MH_WINDOWS(float);
        else if (values_dtype == GRWS_F16) GRWS_MH_WINDOWS(_Float16);
        else GRWS_MH_WINDOWS(__hip_bfloat16);
#undef GRWS_MH_WINDOWS
        GRWS_LAUNCH_CHECK();
        if (any_t && thops[h]) {
            // the hop's slots are still in the workspace: its transposed block
            const int64_t ecap = c.E[h], wcap = c.WT[h];
#define GRWS_MH_T(KERNEL, VT, ...) hipLaunchKernelGGL(KERNEL<VT>, __VA_ARGS__)
#define GRWS_MH_TDISPATCH(KERNEL, ...)                                                  \
    if (values_dtype == GRWS_F32) GRWS_MH_T(KERNEL, float, __VA_ARGS__);                \
    else if (values_dtype == GRWS_F16) GRWS_MH_T(KERNEL, _Float16, __VA_ARGS__);        \
    else GRWS_MH_T(KERNEL, __hip_bfloat16, __VA_ARGS__)
            GRWS_MH_TDISPATCH(mh_tkeys_kernel, dim3(grid_for(ecap)), dim3(kBlk), 0, stream, F0, h, k,
                              w.src_local, w.edge_val, ecap, wcap, w.tka, w.tpa, ctr);
            GRWS_LAUNCH_CHECK();
            bool alt = false;
            GRWS_TRY(radix_sort_pairs(w.tka, w.tpa, w.tkb, w.tpb, ecap, bits_for(wcap + 1), w.sort_ws, w.sort_bytes,
                                      stream, &alt));
            const uint64_t* sk = alt ? w.tkb : w.tka;
            const uint32_t* sp = alt ? w.tpb : w.tpa;
            hipLaunchKernelGGL(mh_tbounds_kernel, dim3(grid_for(ecap + 1)), dim3(kBlk), 0, stream, h, sk, ecap, wcap,
                               w.tstart, ctr);
            GRWS_LAUNCH_CHECK();
            const unsigned tgrid = (unsigned)std::min<int64_t>((wcap + kBlk / kWave - 1) / (kBlk / kWave), 256);
            hipLaunchKernelGGL(mh_tcount_kernel, dim3(tgrid), dim3(kBlk), 0, stream, h, k, w.tstart, sp, tc, wcap,
                               w.wtiles, ctr);
            GRWS_LAUNCH_CHECK();
            GRWS_TRY(scan_i32_to_i64(w.wtiles, t_window_offset[h], wcap, false, w.scan_ws, w.scan_bytes, stream));
            GRWS_MH_TDISPATCH(mh_tfill_kernel, dim3((unsigned)wcap), dim3(kBlk), 0, stream, h, k, w.tstart, sp, wcap,
                              tc, w.src_local, w.edge_val, t_window_offset[h], t_col_indices[h], t_values[h],
                              ctr);
#undef GRWS_MH_TDISPATCH
#undef GRWS_MH_T
            GRWS_LAUNCH_CHECK();
        }
    }
    hipLaunchKernelGGL(mh_finish_kernel, dim3(1), dim3(64), 0, stream, ctr, counts_dev ? counts_dev : w.out, H);
    GRWS_LAUNCH_CHECK();
    if (counts_dev) return GRWS_OK;  // enqueued: the caller reads the counts after the stream's work
    int64_t h_out[5 * kMaxHops + 4];
    GRWS_HIP(hipMemcpyAsync(h_out, w.out, sizeof(int64_t) * (5 * H + 2), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    GRWS_TRY(report((int32_t)h_out[5 * H + 1], "sample_blocks"));
    for (int h = 0; h < H; ++h) {
        counts_out[per_hop * h + 0] = h_out[H + 1 + h];      // edges
        counts_out[per_hop * h + 1] = h_out[h + 1];          // sources (next frontier size)
        counts_out[per_hop * h + 2] = h_out[2 * H + 1 + h];  // tiles
        if (per_hop == 5) {
            counts_out[per_hop * h + 3] = h_out[3 * H + 1 + h];  // tiles of the transposed block
            counts_out[per_hop * h + 4] = h_out[4 * H + 1 + h];  // most tiles in one of its windows
        }
    }
    return GRWS_OK;
}

extern "C" int grws_sample_blocks(const int64_t* indptr, const int32_t* indices, int64_t num_nodes, int64_t nnz,
                                  const int64_t* seeds, int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                                  uint64_t seed, int32_t* node_map, uint32_t* state, int32_t tile_cols,
                                  int32_t values_dtype, int64_t* const* next_frontier,
                                  int64_t* const* window_offset, int32_t* const* col_indices,
                                  void* const* values, void* workspace, size_t workspace_bytes, int64_t* counts_out,
                                  void* stream_) {
    clear_error();
    return sample_blocks_impl(indptr, indices, num_nodes, nnz, seeds, num_seeds, fanouts, num_hops, seed, node_map,
                              state, tile_cols, values_dtype, next_frontier, window_offset, col_indices, values,
                              nullptr, nullptr, nullptr, nullptr, workspace, workspace_bytes, counts_out, 3,
                              nullptr, nullptr, as_stream(stream_));
}

extern "C" int grws_sample_blocks_transposed(const int64_t* indptr, const int32_t* indices, int64_t num_nodes,
                                             int64_t nnz, const int64_t* seeds, int64_t num_seeds,
                                             const int32_t* fanouts, int32_t num_hops, uint64_t seed,
                                             int32_t* node_map, uint32_t* state, int32_t tile_cols,
                                             int32_t values_dtype, int64_t* const* next_frontier,
                                             int64_t* const* window_offset, int32_t* const* col_indices,
                                             void* const* values, const int32_t* transpose_hops,
                                             int64_t* const* t_window_offset, int32_t* const* t_col_indices,
                                             void* const* t_values, void* workspace, size_t workspace_bytes,
                                             int64_t* counts_out, void* stream_) {
    clear_error();
    GRWS_CHECK_ARG(transpose_hops != nullptr, "sample_blocks_transposed: null transpose_hops");
    return sample_blocks_impl(indptr, indices, num_nodes, nnz, seeds, num_seeds, fanouts, num_hops, seed, node_map,
                              state, tile_cols, values_dtype, next_frontier, window_offset, col_indices, values,
                              transpose_hops, t_window_offset, t_col_indices, t_values, workspace, workspace_bytes,
                              counts_out, 5, nullptr, nullptr, as_stream(stream_));
}

extern "C" int grws_sample_blocks_enqueue(const int64_t* indptr, const int32_t* indices, int64_t num_nodes,
                                          int64_t nnz, const int64_t* seeds, int64_t max_seeds,
                                          const int64_t* num_seeds_dev, const int32_t* fanouts, int32_t num_hops,
                                          uint64_t seed, int32_t* node_map, uint32_t* state, int32_t tile_cols,
                                          int32_t values_dtype, int64_t* const* next_frontier,
                                          int64_t* const* window_offset, int32_t* const* col_indices,
                                          void* const* values, const int32_t* transpose_hops,
                                          int64_t* const* t_window_offset, int32_t* const* t_col_indices,
                                          void* const* t_values, void* workspace, size_t workspace_bytes,
                                          int64_t* counts_dev, void* stream_) {
    clear_error();
    GRWS_CHECK_ARG(max_seeds >= 1, "sample_blocks_enqueue: max_seeds must be at least 1");
    GRWS_CHECK_ARG(num_seeds_dev != nullptr && counts_dev != nullptr, "sample_blocks_enqueue: null pointer");
    bool any_t = false;
    for (int h = 0; transpose_hops && h < num_hops && h < kMaxHops; ++h) any_t = any_t || transpose_hops[h];
    return sample_blocks_impl(indptr, indices, num_nodes, nnz, seeds, max_seeds, fanouts, num_hops, seed, node_map,
                              state, tile_cols, values_dtype, next_frontier, window_offset, col_indices, values,
                              any_t ? transpose_hops : nullptr, t_window_offset, t_col_indices, t_values, workspace,
                              workspace_bytes, nullptr, any_t ? 5 : 3, num_seeds_dev, counts_dev,
                              as_stream(stream_));
}

extern "C" int grws_sample_blocks_error(int64_t err) {
    clear_error();
    return report((int32_t)err, "sample_blocks");
}

// ---------------------------------------------------------------------------
// Batched device copies (one launch for many ranges)
// ---------------------------------------------------------------------------
namespace grws {
namespace {

constexpr int kMaxCopyRanges = 32;

struct CopyArgs {
    const char* src[kMaxCopyRanges];
    char* dst[kMaxCopyRanges];
    int64_t first[kMaxCopyRanges + 1];  // first 16-byte unit of each range (prefix over ranges)
    int64_t bytes[kMaxCopyRanges];
    int n;
};

// Unit u of the launch belongs to the range r with first[r] <= u < first[r+1];
// a unit is 16 bytes of its range, the last one possibly shorter (copied
// byte by byte).  Ranges are 16-byte aligned at both ends' bases.
__global__ __launch_bounds__(256) void copy_ranges_kernel(CopyArgs a) {
    const int64_t total = a.first[a.n];
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < total; u += (int64_t)gridDim.x * 256) {
        int r = 0;
        while (u >= a.first[r + 1]) ++r;
        const int64_t off = (u - a.first[r]) * 16;
        const int64_t left = a.bytes[r] - off;
        if (left >= 16) {
            *reinterpret_cast<u32x4_t*>(a.dst[r] + off) = *reinterpret_cast<const u32x4_t*>(a.src[r] + off);
        } else {
            for (int64_t b = 0; b < left; ++b) a.dst[r][off + b] = a.src[r][off + b];
        }
    }
}

struct FillArgs {
    int64_t* dst[kMaxCopyRanges];
    int64_t first[kMaxCopyRanges + 1];  // first element of each range (prefix over ranges)
    int64_t value[kMaxCopyRanges];
    int n;
};

// Element u of the launch belongs to the range r with first[r] <= u < first[r+1].
__global__ __launch_bounds__(256) void fill_ranges_kernel(FillArgs a) {
    const int64_t total = a.first[a.n];
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < total; u += (int64_t)gridDim.x * 256) {
        int r = 0;
        while (u >= a.first[r + 1]) ++r;
        a.dst[r][u - a.first[r]] = a.value[r];
    }
}

}  // namespace
}  // namespace grws

extern "C" int grws_fill_ranges_i64(int64_t* const* dst, const int64_t* count, const int64_t* value, int32_t n,
                                    void* stream_) {
    clear_error();
    GRWS_CHECK_ARG(n >= 0, "fill_ranges: negative count");
    if (n == 0) return GRWS_OK;
    GRWS_CHECK_ARG(dst && count && value, "fill_ranges: null pointer");
    const hipStream_t stream = as_stream(stream_);
    for (int32_t base = 0; base < n; base += kMaxCopyRanges) {
        FillArgs a{};
        a.n = 0;
        a.first[0] = 0;
        for (int32_t i = base; i < n && i < base + kMaxCopyRanges; ++i) {
            GRWS_CHECK_ARG(count[i] >= 0, "fill_ranges: negative length");
            GRWS_CHECK_ARG(count[i] == 0 || dst[i], "fill_ranges: null range");
            GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(dst[i]) % 8 == 0, "fill_ranges: range %d not 8-byte aligned", i);
            a.dst[a.n] = dst[i];
            a.value[a.n] = value[i];
            a.first[a.n + 1] = a.first[a.n] + count[i];
            ++a.n;
        }
        const int64_t total = a.first[a.n];
        if (total == 0) continue;
        const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 4096);
        hipLaunchKernelGGL(fill_ranges_kernel, dim3(grid), dim3(256), 0, stream, a);
        GRWS_LAUNCH_CHECK();
    }
    return GRWS_OK;
}

extern "C" int grws_copy_ranges(const void* const* src, void* const* dst, const int64_t* bytes, int32_t n,
                                void* stream_) {
    clear_error();
    GRWS_CHECK_ARG(n >= 0, "copy_ranges: negative count");
    if (n == 0) return GRWS_OK;
    GRWS_CHECK_ARG(src && dst && bytes, "copy_ranges: null pointer");
    const hipStream_t stream = as_stream(stream_);
    for (int32_t base = 0; base < n; base += kMaxCopyRanges) {
        CopyArgs a{};
        a.n = 0;
        a.first[0] = 0;
        for (int32_t i = base; i < n && i < base + kMaxCopyRanges; ++i) {
            GRWS_CHECK_ARG(bytes[i] >= 0, "copy_ranges: negative length");
            GRWS_CHECK_ARG(bytes[i] == 0 || (src[i] && dst[i]), "copy_ranges: null range");
            GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(src[i]) % 16 == 0 && reinterpret_cast<uintptr_t>(dst[i]) % 16 == 0,
                           "copy_ranges: range %d not 16-byte aligned", i);
            a.src[a.n] = static_cast<const char*>(src[i]);
            a.dst[a.n] = static_cast<char*>(dst[i]);
            a.bytes[a.n] = bytes[i];
            a.first[a.n + 1] = a.first[a.n] + (bytes[i] + 15) / 16;
            ++a.n;
        }
        const int64_t total = a.first[a.n];
        if (total == 0) continue;
        const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 4096);
        hipLaunchKernelGGL(copy_ranges_kernel, dim3(grid), dim3(256), 0, stream, a);
        GRWS_LAUNCH_CHECK();
    }
    return GRWS_OK;
}

// ---------------------------------------------------------------------------
// Row gather (the mini-batch producer's input features)
// ---------------------------------------------------------------------------
// dst[i, :] = src[idx[i], :].  Each work item moves one unit of UB bytes
// (the widest of 16/8/4/2/1 that divides the row length, both pitches and
// both base addresses); the units of a row are consecutive items, so a wave
// reads whole rows (a 256-byte row: 16 lanes of 16 bytes).  Every thread
// handles kGatherUnroll items a grid stride apart and issues all of their
// loads before its stores, to keep many random rows in flight.
namespace grws {
namespace {

constexpr int kGatherBlock = 256;
constexpr int kGatherUnroll = 4;

template <int UB> struct GatherUnit;
template <> struct GatherUnit<16> { typedef u32x4_t T; };
template <> struct GatherUnit<8> { typedef uint64_t T; };
template <> struct GatherUnit<4> { typedef uint32_t T; };
template <> struct GatherUnit<2> { typedef uint16_t T; };
template <> struct GatherUnit<1> { typedef uint8_t T; };

template <int UB, bool IDX64>
__global__ __launch_bounds__(kGatherBlock) void gather_rows_kernel(const char* __restrict__ src, int64_t src_rows,
                                                                   int64_t ld_src, const void* __restrict__ idx,
                                                                   int64_t total, uint32_t upr,
                                                                   char* __restrict__ dst, int64_t ld_dst,
                                                                   int32_t* __restrict__ err) {
    using T = typename GatherUnit<UB>::T;
    const int64_t stride = (int64_t)gridDim.x * kGatherBlock;
    for (int64_t base = (int64_t)blockIdx.x * kGatherBlock + threadIdx.x; base < total;
         base += stride * kGatherUnroll) {
        T v[kGatherUnroll];
        int64_t row[kGatherUnroll];
        uint32_t unit[kGatherUnroll];
        bool in[kGatherUnroll];
        bool bad = false;
#pragma unroll
        for (int j = 0; j < kGatherUnroll; ++j) {
            const int64_t u = base + j * stride;
            in[j] = u < total;
            row[j] = in[j] ? u / upr : 0;
            unit[j] = in[j] ? (uint32_t)(u - row[j] * upr) : 0u;
            const int64_t s = !in[j]   ? 0
                              : IDX64 ? static_cast<const int64_t*>(idx)[row[j]]
                                      : (int64_t) static_cast<const int32_t*>(idx)[row[j]];
            const bool ok = in[j] && s >= 0 && s < src_rows;
            bad |= in[j] && !ok;
            v[j] = ok ? *reinterpret_cast<const T*>(src + s * ld_src + (int64_t)unit[j] * UB) : T{};
        }
#pragma unroll
        for (int j = 0; j < kGatherUnroll; ++j)
            if (in[j]) *reinterpret_cast<T*>(dst + row[j] * ld_dst + (int64_t)unit[j] * UB) = v[j];
        if (bad && err) *err = 1;
    }
}

template <int UB>
void launch_gather_rows(const void* src, int64_t src_rows, int64_t ld_src, const void* idx, bool idx64, int64_t n,
                        int64_t row_bytes, void* dst, int64_t ld_dst, int32_t* err, hipStream_t stream) {
    const int64_t upr = row_bytes / UB;
    const int64_t total = n * upr;
    const int64_t want = (total + (int64_t)kGatherBlock * kGatherUnroll - 1) / ((int64_t)kGatherBlock * kGatherUnroll);
    const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, 65536));
    if (idx64)
        hipLaunchKernelGGL((gather_rows_kernel<UB, true>), dim3(grid), dim3(kGatherBlock), 0, stream,
                           static_cast<const char*>(src), src_rows, ld_src, idx, total, (uint32_t)upr,
                           static_cast<char*>(dst), ld_dst, err);
    else
        hipLaunchKernelGGL((gather_rows_kernel<UB, false>), dim3(grid), dim3(kGatherBlock), 0, stream,
                           static_cast<const char*>(src), src_rows, ld_src, idx, total, (uint32_t)upr,
                           static_cast<char*>(dst), ld_dst, err);
}

}  // namespace
}  // namespace grws

extern "C" int grws_gather_rows(const void* src, int64_t src_rows, int64_t ld_src, const void* idx,
                                int32_t idx_is_i64, int64_t n, int64_t row_bytes, void* dst, int64_t ld_dst,
                                int32_t* err, void* stream_) {
    clear_error();
    GRWS_CHECK_ARG(n >= 0 && src_rows >= 0 && row_bytes >= 0, "gather_rows: negative size");
    if (n == 0 || row_bytes == 0) return GRWS_OK;
    GRWS_CHECK_ARG(src != nullptr && idx != nullptr && dst != nullptr, "gather_rows: null pointer");
    GRWS_CHECK_ARG(ld_src >= row_bytes && ld_dst >= row_bytes, "gather_rows: row pitch below the row length");
    GRWS_CHECK_ARG(row_bytes <= ((int64_t)1 << 31), "gather_rows: rows above 2 GiB");
    const uint64_t align = (uint64_t)row_bytes | (uint64_t)ld_src | (uint64_t)ld_dst | (uint64_t)(uintptr_t)src |
                           (uint64_t)(uintptr_t)dst;
    const hipStream_t stream = as_stream(stream_);
    const bool i64 = idx_is_i64 != 0;
    if ((align & 15) == 0)
        launch_gather_rows<16>(src, src_rows, ld_src, idx, i64, n, row_bytes, dst, ld_dst, err, stream);
    else if ((align & 7) == 0)
        launch_gather_rows<8>(src, src_rows, ld_src, idx, i64, n, row_bytes, dst, ld_dst, err, stream);
    else if ((align & 3) == 0)
        launch_gather_rows<4>(src, src_rows, ld_src, idx, i64, n, row_bytes, dst, ld_dst, err, stream);
    else if ((align & 1) == 0)
        launch_gather_rows<2>(src, src_rows, ld_src, idx, i64, n, row_bytes, dst, ld_dst, err, stream);
    else
        launch_gather_rows<1>(src, src_rows, ld_src, idx, i64, n, row_bytes, dst, ld_dst, err, stream);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

