// Grouped tiles: the BCSR of A re-tiled so that G consecutive row windows
// share their column slabs (gfx950).
//
// A 16-row window multiplies its own distinct columns, 16 per tile.  On a
// graph with community structure neighbouring windows reference mostly the
// same columns, so the SpMM gathers the same X rows once per window.  Here
// the G windows of a group get one sorted list of the union of their
// columns, cut into slabs of 16; for every slab each window keeps a 16x16
// sub-tile holding its values in those columns (zeros elsewhere), packed as
// the SpMM's packed tiles are (per 4-row group a 64-bit mask of the nonzero
// slots and the index of the group's first value).  The grouped SpMM kernel
// then gathers each slab's 16 X rows once and multiplies them by the G
// sub-tiles.
//
// Build, two calls (one host sync, in the first):
//   count: the union's size per group -> slabs per group -> group_offset
//          (kept in the workspace); the nonzero value count; the longest
//          group.  Graphs of at most 2^18 columns: one work-group per group
//          sets a bit per valid slot in an LDS bitmap of all the columns and
//          counts them; wider graphs: the (group, column) key of every valid
//          slot, a stable radix sort, distinct keys ranked.
//   fill:  union columns and every slot's (slab, position) (the bitmap again,
//          its popcount bases giving places; or the sorted ranks), masks by
//          atomic OR, value counts -> scan -> group starts, then every value
//          placed by the popcount of the mask bits below it (deterministic).
#include "grws_internal.h"

namespace grws {
namespace {

constexpr int kBlk = 256;

inline int bits_for(int64_t x) {
    int b = 0;
    while (b < 63 && ((int64_t)1 << b) < x) ++b;
    return b;
}

inline unsigned grid_for(int64_t n, int64_t per_block = kBlk) {
    int64_t g = (n + per_block - 1) / per_block;
    return (unsigned)(g < 1 ? 1 : g);
}

struct GroupShape {
    int64_t n;      // tile slots (T * tc)
    int64_t Q;      // groups
    int G;          // windows per group
    int cbits;      // column bits
    int bits;       // sort key bits: group, column, then the invalid flag
    int64_t scan_n; // longest scan
};

GroupShape group_shape(const grws_bcsr* A, int64_t num_cols, int G) {
    GroupShape s;
    s.n = A->num_tiles * A->tile_cols;
    s.G = G;
    s.Q = (A->num_windows + G - 1) / G;
    s.cbits = bits_for(num_cols > 1 ? num_cols : 2);
    s.bits = bits_for(s.Q > 1 ? s.Q : 2) + s.cbits + 1;
    // sub-tile count scan: slabs <= tiles + groups
    const int64_t subs = (A->num_tiles + s.Q) * G;
    s.scan_n = s.n > subs ? s.n : subs;
    if (s.scan_n < s.Q + 1) s.scan_n = s.Q + 1;
    return s;
}

struct GroupWs {
    uint64_t *ka, *kb;
    uint32_t *va, *vb;
    int32_t* uflag;
    int64_t* uidx;     // exclusive scan of uflag, n + 1
    uint32_t* pos;     // per slot: slab * 16 + position in the slab
    int64_t* gfirst;   // per group: rank of its first distinct column
    int64_t* glast;    // per group: one past its last
    int32_t* gslabs;   // per group: slabs
    int64_t* goff;     // group_offset, Q + 1
    int32_t* scnt;     // per sub-tile: values
    int64_t* soff;     // their exclusive scan
    int64_t* stats;    // [0] nonzero values, [1] longest group (slabs)
    char* sort_ws;
    size_t sort_bytes;
    char* scan_ws;
    size_t scan_bytes;
    bool alt;          // sorted keys in kb/vb
};

template <typename C>
void carve_group(C& cv, const GroupShape& s, GroupWs* w) {
    const int64_t n = s.n > 0 ? s.n : 1;
    w->ka = cv.template take<uint64_t>(n);
    w->kb = cv.template take<uint64_t>(n);
    w->va = cv.template take<uint32_t>(n);
    w->vb = cv.template take<uint32_t>(n);
    w->uflag = cv.template take<int32_t>(n);
    w->uidx = cv.template take<int64_t>(n + 1);
    w->pos = cv.template take<uint32_t>(n);
    w->gfirst = cv.template take<int64_t>(s.Q + 1);
    w->glast = cv.template take<int64_t>(s.Q + 1);
    w->gslabs = cv.template take<int32_t>(s.Q + 1);
    w->goff = cv.template take<int64_t>(s.Q + 1);
    w->stats = cv.template take<int64_t>(4);
    w->sort_bytes = radix_sort_workspace_bytes(n);
    w->sort_ws = cv.template take<char>(w->sort_bytes);
    w->scan_bytes = scan_workspace_bytes(s.scan_n);
    w->scan_ws = cv.template take<char>(w->scan_bytes);
    w->scnt = nullptr;
    w->soff = nullptr;
}

struct NullCarver {
    Sizer s;
    template <typename T>
    T* take(size_t k) {
        s.take<T>(k);
        return nullptr;
    }
};

// 16-bit value bits of slot (t, r, c): nonzero bits are kept (as the packed
// tiles keep them).
__device__ __forceinline__ uint32_t value_bits(const uint16_t* __restrict__ vals, int64_t t, int r, int c, int tc) {
    return vals[(t * 16 + r) * tc + c];
}

// The window of every tile (twin), one work-group per window; the map starts
// zeroed, so tiles outside every window (only from a malformed
// window_offset) belong to window 0.
__global__ __launch_bounds__(256) void grp_tile_window_kernel(const int64_t* __restrict__ win_off, int64_t W,
                                                              int64_t T, int32_t* __restrict__ twin) {
    for (int64_t w = blockIdx.x; w < W; w += gridDim.x) {
        const int64_t a = win_off[w], e = win_off[w + 1];
        const int64_t t0 = a < 0 ? 0 : (a > T ? T : a);
        const int64_t t1 = e < t0 ? t0 : (e > T ? T : e);
        for (int64_t t = t0 + threadIdx.x; t < t1; t += blockDim.x) twin[t] = (int32_t)w;
    }
}

// Key of every slot: (group << cbits | column), or the invalid flag for a
// padding slot or a column outside [0, num_cols).
__global__ void grp_keys_kernel(const int32_t* __restrict__ twin, const int32_t* __restrict__ cols,
                                int64_t n, int tc, int64_t num_cols, int G, int cbits, int vbit,
                                uint64_t* __restrict__ keys, uint32_t* __restrict__ pay) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int32_t c = cols[i];
    uint64_t k = 1ull << vbit;
    if (c >= 0 && (int64_t)c < num_cols) {
        const int64_t w = twin[i / tc];
        k = ((uint64_t)(w / G) << cbits) | (uint64_t)c;
    }
    keys[i] = k;
    pay[i] = (uint32_t)i;
}

__global__ void grp_unique_kernel(const uint64_t* __restrict__ keys, int64_t n, int vbit, int32_t* __restrict__ uflag) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t k = keys[i];
    uflag[i] = ((k >> vbit) == 0 && (i == 0 || keys[i - 1] != k)) ? 1 : 0;
}

// First and one-past-last distinct rank of every group present.
__global__ void grp_bounds_kernel(const uint64_t* __restrict__ keys, int64_t n, int vbit, int cbits,
                                  const int32_t* __restrict__ uflag, const int64_t* __restrict__ uidx,
                                  int64_t* __restrict__ gfirst, int64_t* __restrict__ glast) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t k = keys[i];
    if ((k >> vbit) != 0) return;
    const uint64_t q = k >> cbits;
    if (i == 0 || (keys[i - 1] >> cbits) != q) gfirst[q] = uidx[i];
    if (i == n - 1 || (keys[i + 1] >> cbits) != q) glast[q] = uidx[i] + uflag[i];
}

__global__ void grp_slabs_kernel(const int64_t* __restrict__ gfirst, const int64_t* __restrict__ glast, int64_t Q,
                                 int32_t* __restrict__ gslabs, int64_t* __restrict__ stats) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    const int64_t u = glast[q] - gfirst[q];
    const int32_t s = (int32_t)((u + 15) / 16);
    gslabs[q] = s;
    if (s > 0) atomicMax((unsigned long long*)&stats[1], (unsigned long long)s);
}

// Nonzero values at valid columns.  Each wave walks tiles t = its global
// wave index + k * (all waves) (lane l: row l / 4, columns 4 (l % 4) .. +3
// at tc 16, or row l / 4, columns 2 (l % 4) .. +1 at tc 8) and adds its
// count once at the end: one atomic per wave, not per tile.
__global__ __launch_bounds__(256) void grp_count_values_kernel(const int32_t* __restrict__ cols,
                                                               const uint16_t* __restrict__ vals, int64_t T, int tc,
                                                               int64_t num_cols, int64_t* __restrict__ stats) {
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * 4;
    const int per = 16 * tc / 64;  // slots per lane: 4 (tc 16) or 2 (tc 8)
    int64_t cnt = 0;
    for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < T; t += nw) {  // uniform per wave
        for (int j = 0; j < per; ++j) {
            const int slot = lane * per + j;
            const int r = slot / tc, c = slot % tc;
            const int32_t col = cols[t * tc + c];
            if (col >= 0 && (int64_t)col < num_cols && value_bits(vals, t, r, c, tc) != 0) ++cnt;
        }
    }
    for (int d = 32; d > 0; d >>= 1) cnt += __shfl_xor(cnt, d, 64);
    if (lane == 0 && cnt) atomicAdd((unsigned long long*)&stats[0], (unsigned long long)cnt);
}

// The same count from 16 bytes of values a lane (values 16-byte aligned):
// chunk x holds slots 8 (x % tpb) .. + 7 of tile x / tpb (tpb = 2 tc chunks
// a tile); one atomic per wave.
__global__ __launch_bounds__(256) void grp_count_values16_kernel(const int32_t* __restrict__ cols,
                                                                 const uint16_t* __restrict__ vals, int64_t T, int tc,
                                                                 int64_t num_cols, int64_t* __restrict__ stats) {
    const int tpb = 2 * tc;
    const int64_t nch = T * tpb;
    int64_t cnt = 0;
    for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < nch; x += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = x / tpb;
        const int s0 = (int)(x % tpb) * 8;
        const uint4 raw = reinterpret_cast<const uint4*>(vals)[x];
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t v = (w4[k >> 1] >> (16 * (k & 1))) & 0xffffu;
            const int32_t col = cols[t * tc + (s0 + k) % tc];
            cnt += (v != 0 && col >= 0 && (int64_t)col < num_cols) ? 1 : 0;
        }
    }
    for (int d = 32; d > 0; d >>= 1) cnt += __shfl_xor(cnt, d, 64);
    if ((threadIdx.x & 63) == 0 && cnt) atomicAdd((unsigned long long*)&stats[0], (unsigned long long)cnt);
}

// Every valid sorted slot: its (slab, position); the group's union column.
__global__ void grp_place_kernel(const uint64_t* __restrict__ keys, const uint32_t* __restrict__ pay, int64_t n,
                                 int vbit, int cbits, const int32_t* __restrict__ uflag,
                                 const int64_t* __restrict__ uidx, const int64_t* __restrict__ gfirst,
                                 const int64_t* __restrict__ goff, uint32_t* __restrict__ pos,
                                 int32_t* __restrict__ gcols) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t k = keys[i];
    if ((k >> vbit) != 0) return;
    const uint64_t q = k >> cbits;
    const int64_t u = uidx[i] + uflag[i] - 1;  // rank of this distinct (group, column)
    const int64_t p = u - gfirst[q];
    const int64_t slab = goff[q] + p / 16;
    const int cc = (int)(p % 16);
    pos[pay[i]] = (uint32_t)(slab * 16 + cc);
    if (uflag[i]) gcols[slab * 16 + cc] = (int32_t)(k & ((1ull << cbits) - 1ull));
}

// Sub-tile slot of a nonzero at (tile t, row r, column slot c): header word
// and bit.  Row group g = r / 4 holds mask bits (r % 4) * 16 + position.
struct SubSlot {
    int64_t sub;  // slab * G + window in group
    int g, bit;
};

__device__ __forceinline__ SubSlot sub_slot(const uint32_t* __restrict__ pos, int64_t w, int G, int64_t t, int r,
                                            int c, int tc) {
    const uint32_t p = pos[t * tc + c];
    SubSlot s;
    s.sub = (int64_t)(p >> 4) * G + (w % G);
    s.g = r >> 2;
    s.bit = (r & 3) * 16 + (int)(p & 15u);
    return s;
}

// Masks (atomic OR; the header starts zeroed).  One wave per tile.
__global__ __launch_bounds__(256) void grp_mask_kernel(const int32_t* __restrict__ twin,
                                                       const int32_t* __restrict__ cols,
                                                       const uint16_t* __restrict__ vals, int64_t T, int tc,
                                                       int64_t num_cols, int G, const uint32_t* __restrict__ pos,
                                                       uint32_t* __restrict__ hdr) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const int64_t w = twin[t];
    const int per = 16 * tc / 64;
    for (int j = 0; j < per; ++j) {
        const int slot = lane * per + j;
        const int r = slot / tc, c = slot % tc;
        const int32_t col = cols[t * tc + c];
        if (col < 0 || (int64_t)col >= num_cols || value_bits(vals, t, r, c, tc) == 0) continue;
        const SubSlot s = sub_slot(pos, w, G, t, r, c, tc);
        atomicOr(&hdr[s.sub * 12 + s.g * 3 + (s.bit >> 5)], 1u << (s.bit & 31));
    }
}

// Graphs of at most kUnionCols columns (c2, c3) skip the sort: one
// work-group per group sets a bit per valid tile slot in an LDS bitmap of
// [0, num_cols); its popcount is the union's size (count), and popcount
// bases give every column its place in the union (fill).  The group's tiles
// are contiguous: those of windows [qG, qG + G).
constexpr int64_t kUnionCols = 1 << 18;   // bitmap bits: 32 KB
constexpr int kUnionWords = (int)(kUnionCols / 32);
constexpr int kUnionBase = 4;             // words per popcount base

__device__ __forceinline__ void union_bitmap(const int64_t* __restrict__ win_off, int64_t W, int64_t T,
                                             const int32_t* __restrict__ cols, int tc, int64_t num_cols, int G,
                                             int64_t q, uint32_t* bm, int nwords, int64_t* x0, int64_t* x1) {
    const int64_t wa = q * G, wb = (q + 1) * G < W ? (q + 1) * G : W;
    const int64_t a = win_off[wa], e = win_off[wb];
    const int64_t t0 = a < 0 ? 0 : (a > T ? T : a);
    const int64_t t1 = e < t0 ? t0 : (e > T ? T : e);
    for (int x = threadIdx.x; x < nwords; x += blockDim.x) bm[x] = 0;
    __syncthreads();
    for (int64_t x = t0 * tc + threadIdx.x; x < t1 * tc; x += blockDim.x) {
        const int32_t c = cols[x];
        if (c >= 0 && (int64_t)c < num_cols) atomicOr(&bm[c >> 5], 1u << (c & 31));
    }
    __syncthreads();
    *x0 = t0 * tc;
    *x1 = t1 * tc;
}

__global__ __launch_bounds__(512) void grp_union_count_kernel(const int64_t* __restrict__ win_off, int64_t W, int64_t T,
                                                              const int32_t* __restrict__ cols, int tc,
                                                              int64_t num_cols, int G, int64_t Q,
                                                              int32_t* __restrict__ gslabs, int64_t* __restrict__ stats) {
    __shared__ uint32_t bm[kUnionWords];
    __shared__ int64_t tmp[512 / 64 + 1];
    const int nwords = (int)((num_cols + 31) / 32);
    for (int64_t q = blockIdx.x; q < Q; q += gridDim.x) {  // uniform over the work-group
        int64_t x0, x1;
        union_bitmap(win_off, W, T, cols, tc, num_cols, G, q, bm, nwords, &x0, &x1);
        int c = 0;
        for (int x = threadIdx.x; x < nwords; x += 512) c += __popc(bm[x]);
        int64_t tot;
        block_incl_scan<512>(c, tmp, &tot);
        if (threadIdx.x == 0) {
            const int32_t sl = (int32_t)((tot + 15) / 16);
            gslabs[q] = sl;
            if (sl > 0) atomicMax((unsigned long long*)&stats[1], (unsigned long long)sl);
        }
        __syncthreads();  // the bitmap is rewritten for the next group
    }
}

__global__ __launch_bounds__(512) void grp_union_fill_kernel(const int64_t* __restrict__ win_off, int64_t W, int64_t T,
                                                             const int32_t* __restrict__ cols, int tc, int64_t num_cols,
                                                             int G, int64_t Q, const int64_t* __restrict__ goff,
                                                             uint32_t* __restrict__ pos, int32_t* __restrict__ gcols) {
    __shared__ uint32_t bm[kUnionWords];
    __shared__ uint32_t base[kUnionWords / kUnionBase];
    __shared__ int64_t tmp[512 / 64 + 1];
    const int nwords = (int)((num_cols + 31) / 32);
    const int nbase = (nwords + kUnionBase - 1) / kUnionBase;
    for (int64_t q = blockIdx.x; q < Q; q += gridDim.x) {  // uniform over the work-group
        int64_t x0, x1;
        union_bitmap(win_off, W, T, cols, tc, num_cols, G, q, bm, nwords, &x0, &x1);
        {  // bases: each thread a contiguous run of entries, one block scan
            const int E = (nbase + 511) / 512;
            const int a0 = min((int)threadIdx.x * E, nbase), a1 = min(a0 + E, nbase);
            int sum = 0;
            for (int b = a0; b < a1; ++b)
                for (int k = 0; k < kUnionBase; ++k)
                    if (b * kUnionBase + k < nwords) sum += __popc(bm[b * kUnionBase + k]);
            int64_t tot;
            int run = (int)(block_incl_scan<512>(sum, tmp, &tot) - sum);
            for (int b = a0; b < a1; ++b) {
                base[b] = (uint32_t)run;
                for (int k = 0; k < kUnionBase; ++k)
                    if (b * kUnionBase + k < nwords) run += __popc(bm[b * kUnionBase + k]);
            }
        }
        __syncthreads();
        const int64_t s16 = goff[q] * 16;  // the group's first slot position
        auto place = [&](int32_t c) -> uint32_t {
            const int wd = c >> 5;
            uint32_t p = base[wd / kUnionBase] + __popc(bm[wd] & ((1u << (c & 31)) - 1u));
            for (int k = wd - wd % kUnionBase; k < wd; ++k) p += __popc(bm[k]);
            return p;
        };
        // the union's columns at their places
        for (int x = threadIdx.x; x < nwords; x += 512) {
            uint32_t v = bm[x];
            while (v) {
                const int b = __ffs(v) - 1;
                v &= v - 1;
                const int32_t c = x * 32 + b;
                gcols[s16 + place(c)] = c;
            }
        }
        // every valid slot's (slab, position)
        for (int64_t x = x0 + threadIdx.x; x < x1; x += 512) {
            const int32_t c = cols[x];
            if (c >= 0 && (int64_t)c < num_cols) pos[x] = (uint32_t)(s16 + place(c));
        }
        __syncthreads();  // the bitmap is rewritten for the next group
    }
}

// The masks and the values with each lane's PER slots (PER = 16 tc / 64: one
// row, PER consecutive columns) read by one vector load each of values,
// columns and positions (values 8-byte aligned at PER 4, 4-byte at PER 2;
// the host checks), then every slot's header words loaded together.
template <int PER>
struct SlotVecs {
    uint32_t v[PER];
    int32_t c[PER];
    uint32_t p[PER];
};
template <int PER>
__device__ __forceinline__ SlotVecs<PER> load_slots(const int32_t* __restrict__ cols, const uint16_t* __restrict__ vals,
                                                    const uint32_t* __restrict__ pos, int64_t t, int tc, int lane) {
    const int slot0 = lane * PER, r = slot0 / tc, c0 = slot0 % tc;
    SlotVecs<PER> o;
    if constexpr (PER == 4) {
        const uint2 vv = *reinterpret_cast<const uint2*>(vals + (t * 16 + r) * tc + c0);
        const int4 cc = *reinterpret_cast<const int4*>(cols + t * tc + c0);
        const uint4 pp = *reinterpret_cast<const uint4*>(pos + t * tc + c0);
        o.v[0] = vv.x & 0xffffu; o.v[1] = vv.x >> 16; o.v[2] = vv.y & 0xffffu; o.v[3] = vv.y >> 16;
        o.c[0] = cc.x; o.c[1] = cc.y; o.c[2] = cc.z; o.c[3] = cc.w;
        o.p[0] = pp.x; o.p[1] = pp.y; o.p[2] = pp.z; o.p[3] = pp.w;
    } else {
        const uint32_t vv = *reinterpret_cast<const uint32_t*>(vals + (t * 16 + r) * tc + c0);
        const int2 cc = *reinterpret_cast<const int2*>(cols + t * tc + c0);
        const uint2 pp = *reinterpret_cast<const uint2*>(pos + t * tc + c0);
        o.v[0] = vv & 0xffffu; o.v[1] = vv >> 16;
        o.c[0] = cc.x; o.c[1] = cc.y;
        o.p[0] = pp.x; o.p[1] = pp.y;
    }
    return o;
}

template <int PER>
__global__ __launch_bounds__(256) void grp_mask_vec_kernel(const int32_t* __restrict__ twin,
                                                           const int32_t* __restrict__ cols,
                                                           const uint16_t* __restrict__ vals, int64_t T, int tc,
                                                           int64_t num_cols, int G, const uint32_t* __restrict__ pos,
                                                           uint32_t* __restrict__ hdr) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const int64_t w = twin[t];
    const SlotVecs<PER> sv = load_slots<PER>(cols, vals, pos, t, tc, lane);
    const int r = (lane * PER) / tc;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        if (sv.c[k] < 0 || (int64_t)sv.c[k] >= num_cols || sv.v[k] == 0) continue;
        const int64_t sub = (int64_t)(sv.p[k] >> 4) * G + (w % G);
        const int bit = (r & 3) * 16 + (int)(sv.p[k] & 15u);
        atomicOr(&hdr[sub * 12 + (r >> 2) * 3 + (bit >> 5)], 1u << (bit & 31));
    }
}

template <int PER>
__global__ __launch_bounds__(256) void grp_values_vec_kernel(const int32_t* __restrict__ twin,
                                                             const int32_t* __restrict__ cols,
                                                             const uint16_t* __restrict__ vals, int64_t T, int tc,
                                                             int64_t num_cols, int G, const uint32_t* __restrict__ pos,
                                                             const uint32_t* __restrict__ hdr,
                                                             uint16_t* __restrict__ out, int64_t num_values) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const int64_t w = twin[t];
    const SlotVecs<PER> sv = load_slots<PER>(cols, vals, pos, t, tc, lane);
    const int r = (lane * PER) / tc;
    bool ok[PER];
    uint32_t h0[PER], h1[PER], h2[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        ok[k] = sv.c[k] >= 0 && (int64_t)sv.c[k] < num_cols && sv.v[k] != 0;
        // an invalid slot's position was never written: no address from it
        const int64_t sub = ok[k] ? (int64_t)(sv.p[k] >> 4) * G + (w % G) : 0;
        const uint32_t* h = hdr + sub * 12 + (r >> 2) * 3;
        h0[k] = ok[k] ? h[0] : 0u;
        h1[k] = ok[k] ? h[1] : 0u;
        h2[k] = ok[k] ? h[2] : 0u;
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        if (!ok[k]) continue;
        const int bit = (r & 3) * 16 + (int)(sv.p[k] & 15u);
        const uint64_t m = ((uint64_t)h1[k] << 32) | h0[k];
        const uint64_t below = bit ? (m & ((1ull << bit) - 1ull)) : 0ull;
        const int64_t at = (int64_t)h2[k] + __popcll(below);
        if (at < num_values) out[at] = (uint16_t)sv.v[k];
    }
}

__global__ void grp_sub_count_kernel(const uint32_t* __restrict__ hdr, int64_t nsub, int32_t* __restrict__ scnt) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nsub) return;
    int c = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) c += __popc(hdr[i * 12 + g * 3]) + __popc(hdr[i * 12 + g * 3 + 1]);
    scnt[i] = c;
}

__global__ void grp_sub_start_kernel(uint32_t* __restrict__ hdr, int64_t nsub, const int64_t* __restrict__ soff) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nsub) return;
    uint32_t run = (uint32_t)soff[i];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        hdr[i * 12 + g * 3 + 2] = run;
        run += __popc(hdr[i * 12 + g * 3]) + __popc(hdr[i * 12 + g * 3 + 1]);
    }
}

// Every nonzero to its place: the group start plus the mask bits below it.
__global__ __launch_bounds__(256) void grp_values_kernel(const int32_t* __restrict__ twin,
                                                         const int32_t* __restrict__ cols,
                                                         const uint16_t* __restrict__ vals, int64_t T, int tc,
                                                         int64_t num_cols, int G, const uint32_t* __restrict__ pos,
                                                         const uint32_t* __restrict__ hdr, uint16_t* __restrict__ out,
                                                         int64_t num_values) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const int64_t w = twin[t];
    const int per = 16 * tc / 64;
    for (int j = 0; j < per; ++j) {
        const int slot = lane * per + j;
        const int r = slot / tc, c = slot % tc;
        const int32_t col = cols[t * tc + c];
        if (col < 0 || (int64_t)col >= num_cols) continue;
        const uint32_t v = value_bits(vals, t, r, c, tc);
        if (v == 0) continue;
        const SubSlot s = sub_slot(pos, w, G, t, r, c, tc);
        const uint32_t* h = hdr + s.sub * 12 + s.g * 3;
        const uint64_t m = ((uint64_t)h[1] << 32) | h[0];
        const uint64_t below = s.bit ? (m & ((1ull << s.bit) - 1ull)) : 0ull;
        const int64_t at = (int64_t)h[2] + __popcll(below);
        if (at < num_values) out[at] = (uint16_t)v;
    }
}

__global__ void copy_i64_dev_kernel(const int64_t* __restrict__ a, int64_t n, int64_t* __restrict__ b) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) b[i] = a[i];
}

int check_group_args(const grws_bcsr* A, int64_t num_cols, int32_t G) {
    GRWS_CHECK_ARG(A != nullptr, "group_tiles: null graph");
    GRWS_CHECK_ARG(A->tile_rows == 16 && (A->tile_cols == 16 || A->tile_cols == 8),
                   "group_tiles: tiles must be 16x16 or 16x8");
    if (A->values_dtype != GRWS_F16 && A->values_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "group_tiles: values must be F16 or BF16");
    GRWS_CHECK_ARG(G == 2 || G == 4 || G == 8, "group_tiles: group_size must be 2, 4 or 8 (got %d)", G);
    GRWS_CHECK_ARG(A->num_windows >= 0 && A->num_tiles >= 0 && num_cols >= 0, "group_tiles: negative size");
    GRWS_CHECK_ARG(A->num_tiles * A->tile_cols < ((int64_t)1 << 32), "group_tiles: more than 2^32 tile slots");
    GRWS_CHECK_ARG(num_cols <= INT32_MAX, "group_tiles: num_cols exceeds int32 column ids");
    if (A->num_tiles > 0)
        GRWS_CHECK_ARG(A->window_offset && A->col_indices && A->values, "group_tiles: null arrays");
    return GRWS_OK;
}

}  // namespace
}  // namespace grws

using namespace grws;

extern "C" size_t grws_group_tiles_workspace_bytes(const grws_bcsr* A, int64_t num_cols, int32_t group_size) {
    if (!A || A->num_windows < 0 || A->num_tiles < 0 || num_cols < 0) return 0;
    if (group_size != 2 && group_size != 4 && group_size != 8) return 0;
    const GroupShape s = group_shape(A, num_cols, group_size);
    NullCarver nc;
    GroupWs w;
    carve_group(nc, s, &w);
    // sub-tile counts and offsets (at most (tiles + groups) * G sub-tiles)
    const int64_t subs = (A->num_tiles + s.Q) * group_size;
    nc.s.take<int32_t>(subs + 1);
    nc.s.take<int64_t>(subs + 2);
    return nc.s.used + 256;
}

extern "C" int grws_group_tiles_count(const grws_bcsr* A, int64_t num_cols, int32_t group_size, void* workspace,
                                      size_t workspace_bytes, int64_t* num_slabs, int64_t* num_values,
                                      int64_t* max_group_slabs, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_group_args(A, num_cols, group_size));
    GRWS_CHECK_ARG(num_slabs && num_values && max_group_slabs, "group_tiles_count: null output");
    const GroupShape s = group_shape(A, num_cols, group_size);
    Carver cv(workspace, workspace_bytes);
    GroupWs w;
    carve_group(cv, s, &w);
    if (!cv.ok)
        return set_error(GRWS_E_CAPACITY, "group_tiles: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const int vbit = s.bits - 1;
    const int tc = A->tile_cols;
    GRWS_TRY(fill_i64(w.gfirst, s.Q + 1, 0, stream));
    GRWS_TRY(fill_i64(w.glast, s.Q + 1, 0, stream));
    GRWS_TRY(fill_i64(w.stats, 4, 0, stream));
    w.alt = false;
    const bool uni = num_cols <= kUnionCols;  // union bitmaps instead of the sort (the fill decides alike)
    if (s.n > 0 && uni) {
        hipLaunchKernelGGL(grp_union_count_kernel, dim3((unsigned)std::min<int64_t>(s.Q, 4096)), dim3(512), 0, stream,
                           A->window_offset, A->num_windows, A->num_tiles, A->col_indices, tc, num_cols, group_size,
                           s.Q, w.gslabs, w.stats);
        GRWS_LAUNCH_CHECK();
    }
    if (s.n > 0 && !uni) {
        // each tile's window, in pos (the fill's array, unused until then)
        int32_t* twin = reinterpret_cast<int32_t*>(w.pos);
        GRWS_TRY(fill_i32(twin, A->num_tiles, 0, stream));
        hipLaunchKernelGGL(grp_tile_window_kernel, dim3(grid_for(A->num_windows, 1) < 8192u ? grid_for(A->num_windows, 1) : 8192u),
                           dim3(256), 0, stream, A->window_offset, A->num_windows, A->num_tiles, twin);
        GRWS_LAUNCH_CHECK();
        hipLaunchKernelGGL(grp_keys_kernel, dim3(grid_for(s.n)), dim3(kBlk), 0, stream, twin, A->col_indices, s.n,
                           tc, num_cols, group_size, s.cbits, vbit, w.ka, w.va);
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(radix_sort_pairs(w.ka, w.va, w.kb, w.vb, s.n, s.bits, w.sort_ws, w.sort_bytes, stream, &w.alt));
        const uint64_t* k = w.alt ? w.kb : w.ka;
        hipLaunchKernelGGL(grp_unique_kernel, dim3(grid_for(s.n)), dim3(kBlk), 0, stream, k, s.n, vbit, w.uflag);
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(scan_i32_to_i64(w.uflag, w.uidx, s.n, false, w.scan_ws, w.scan_bytes, stream));
        hipLaunchKernelGGL(grp_bounds_kernel, dim3(grid_for(s.n)), dim3(kBlk), 0, stream, k, s.n, vbit, s.cbits,
                           w.uflag, w.uidx, w.gfirst, w.glast);
        GRWS_LAUNCH_CHECK();
    }
    if (s.n > 0) {
        if ((reinterpret_cast<uintptr_t>(A->values) & 15) == 0) {
            const int64_t nch = A->num_tiles * 2 * tc;
            const unsigned cgrid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((nch + 255) / 256, 16384));
            hipLaunchKernelGGL(grp_count_values16_kernel, dim3(cgrid), dim3(256), 0, stream, A->col_indices,
                               static_cast<const uint16_t*>(A->values), A->num_tiles, tc, num_cols, w.stats);
        } else {
            const unsigned cgrid = grid_for(A->num_tiles, 4) < 8192u ? grid_for(A->num_tiles, 4) : 8192u;
            hipLaunchKernelGGL(grp_count_values_kernel, dim3(cgrid), dim3(256), 0, stream, A->col_indices,
                               static_cast<const uint16_t*>(A->values), A->num_tiles, tc, num_cols, w.stats);
        }
        GRWS_LAUNCH_CHECK();
    }
    if (!uni || s.n == 0) {
        hipLaunchKernelGGL(grp_slabs_kernel, dim3(grid_for(s.Q)), dim3(kBlk), 0, stream, w.gfirst, w.glast, s.Q,
                           w.gslabs, w.stats);
        GRWS_LAUNCH_CHECK();
    }
    GRWS_TRY(scan_i32_to_i64(w.gslabs, w.goff, s.Q, false, w.scan_ws, w.scan_bytes, stream));
    int64_t h[3] = {0, 0, 0};
    GRWS_HIP(hipMemcpyAsync(&h[0], w.goff + s.Q, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&h[1], w.stats, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    *num_slabs = h[0];
    *num_values = h[1];
    *max_group_slabs = h[2];
    if (h[0] * 16 >= ((int64_t)1 << 32))
        return set_error(GRWS_E_CAPACITY, "group_tiles: %lld slabs exceed 32-bit slot positions", (long long)h[0]);
    return GRWS_OK;
}

extern "C" int grws_group_tiles_fill(const grws_bcsr* A, int64_t num_cols, int32_t group_size, int64_t num_slabs,
                                     int64_t* group_offset, int32_t* col_indices, uint32_t* header, void* values,
                                     int64_t num_values, void* workspace, size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_group_args(A, num_cols, group_size));
    const GroupShape s = group_shape(A, num_cols, group_size);
    GRWS_CHECK_ARG(num_slabs >= 0 && num_slabs <= A->num_tiles + s.Q, "group_tiles_fill: bad num_slabs %lld",
                   (long long)num_slabs);
    GRWS_CHECK_ARG(num_values >= 0, "group_tiles_fill: negative num_values");
    GRWS_CHECK_ARG(group_offset != nullptr, "group_tiles_fill: null group_offset");
    if (num_slabs > 0) GRWS_CHECK_ARG(col_indices && header, "group_tiles_fill: null outputs");
    if (num_values > 0) GRWS_CHECK_ARG(values != nullptr, "group_tiles_fill: null values");
    Carver cv(workspace, workspace_bytes);
    GroupWs w;
    carve_group(cv, s, &w);
    const int64_t nsub = num_slabs * group_size;
    w.scnt = cv.take<int32_t>((A->num_tiles + s.Q) * group_size + 1);
    w.soff = cv.take<int64_t>((A->num_tiles + s.Q) * group_size + 2);
    if (!cv.ok)
        return set_error(GRWS_E_CAPACITY, "group_tiles: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const int vbit = s.bits - 1;
    const int tc = A->tile_cols;
    // the count pass's sort result: the pass count decides the buffer
    const int passes = (s.bits + 7) / 8;
    const bool alt = s.n > 1 && (passes & 1);
    const uint64_t* k = alt ? w.kb : w.ka;
    const uint32_t* v = alt ? w.vb : w.va;
    hipLaunchKernelGGL(copy_i64_dev_kernel, dim3(grid_for(s.Q + 1)), dim3(kBlk), 0, stream, w.goff, s.Q + 1,
                       group_offset);
    GRWS_LAUNCH_CHECK();
    if (num_slabs == 0) return GRWS_OK;
    GRWS_TRY(fill_i32(col_indices, num_slabs * 16, -1, stream));
    GRWS_TRY(fill_bytes_zero(header, (size_t)nsub * 12 * sizeof(uint32_t), stream));
    if (s.n == 0) return GRWS_OK;
    if (num_cols <= kUnionCols) {  // as the count decided
        hipLaunchKernelGGL(grp_union_fill_kernel, dim3((unsigned)std::min<int64_t>(s.Q, 4096)), dim3(512), 0, stream,
                           A->window_offset, A->num_windows, A->num_tiles, A->col_indices, tc, num_cols, group_size,
                           s.Q, w.goff, w.pos, col_indices);
    } else {
        hipLaunchKernelGGL(grp_place_kernel, dim3(grid_for(s.n)), dim3(kBlk), 0, stream, k, v, s.n, vbit, s.cbits,
                           w.uflag, w.uidx, w.gfirst, w.goff, w.pos, col_indices);
    }
    GRWS_LAUNCH_CHECK();
    const uint16_t* vals = static_cast<const uint16_t*>(A->values);
    // each tile's window, in uflag (spent once the slots are placed)
    int32_t* twin = w.uflag;
    GRWS_TRY(fill_i32(twin, A->num_tiles, 0, stream));
    hipLaunchKernelGGL(grp_tile_window_kernel, dim3(grid_for(A->num_windows, 1) < 8192u ? grid_for(A->num_windows, 1) : 8192u),
                       dim3(256), 0, stream, A->window_offset, A->num_windows, A->num_tiles, twin);
    GRWS_LAUNCH_CHECK();
    // vector loads when the values are 8-byte aligned (tc 16) or 4-byte (tc 8)
    // and the columns 16-byte aligned
    const bool vec = (reinterpret_cast<uintptr_t>(vals) & (tc == 16 ? 7 : 3)) == 0 &&
                     (reinterpret_cast<uintptr_t>(A->col_indices) & 15) == 0;
    if (vec && tc == 16)
        hipLaunchKernelGGL(grp_mask_vec_kernel<4>, dim3(grid_for(A->num_tiles, 4)), dim3(256), 0, stream, twin,
                           A->col_indices, vals, A->num_tiles, tc, num_cols, (int)group_size, w.pos, header);
    else if (vec)
        hipLaunchKernelGGL(grp_mask_vec_kernel<2>, dim3(grid_for(A->num_tiles, 4)), dim3(256), 0, stream, twin,
                           A->col_indices, vals, A->num_tiles, tc, num_cols, (int)group_size, w.pos, header);
    else
        hipLaunchKernelGGL(grp_mask_kernel, dim3(grid_for(A->num_tiles, 4)), dim3(256), 0, stream, twin,
                           A->col_indices, vals, A->num_tiles, tc, num_cols, (int)group_size, w.pos, header);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(grp_sub_count_kernel, dim3(grid_for(nsub)), dim3(kBlk), 0, stream, header, nsub, w.scnt);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(w.scnt, w.soff, nsub, false, w.scan_ws, w.scan_bytes, stream));
    hipLaunchKernelGGL(grp_sub_start_kernel, dim3(grid_for(nsub)), dim3(kBlk), 0, stream, header, nsub, w.soff);
    GRWS_LAUNCH_CHECK();
    if (vec && tc == 16)
        hipLaunchKernelGGL(grp_values_vec_kernel<4>, dim3(grid_for(A->num_tiles, 4)), dim3(256), 0, stream, twin,
                           A->col_indices, vals, A->num_tiles, tc, num_cols, (int)group_size, w.pos, header,
                           static_cast<uint16_t*>(values), num_values);
    else if (vec)
        hipLaunchKernelGGL(grp_values_vec_kernel<2>, dim3(grid_for(A->num_tiles, 4)), dim3(256), 0, stream, twin,
                           A->col_indices, vals, A->num_tiles, tc, num_cols, (int)group_size, w.pos, header,
                           static_cast<uint16_t*>(values), num_values);
    else
        hipLaunchKernelGGL(grp_values_kernel, dim3(grid_for(A->num_tiles, 4)), dim3(256), 0, stream, twin,
                           A->col_indices, vals, A->num_tiles, tc, num_cols, (int)group_size, w.pos, header,
                           static_cast<uint16_t*>(values), num_values);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}
