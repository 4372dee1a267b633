// Window top-K sampling of a BCSR graph (gfx950): the reference-compatible
// mode of core_lib.sample_all_layers.
//
// Replaces, with the same results:
//   prepare_windows_and_masks          sampling_wrapper.cu:283-347
//   warp_centric_find_top_k_kernel     sampling.cuh:65-448
//   build_col_to_val_map_kernel + scan sampling.cuh:707-773, sampling_wrapper.cu:160-204
//   recompress_sampled_bcsr_kernel     sampling.cuh:471-579
//
// Semantics (per active window, all of it determined by the reference):
//   * every column slot c != -1 of the window scores each of its tile_rows
//     values v:  non-HACS  s = trunc(fma(10, |v|, 1) * 1000)
//                HACS      s = trunc((fma(beta, |v|, alpha) * q[col]
//                                     [+ delta if col in the window's part])
//                                    * scale)
//     (sampling.cuh:251-275); a value with s <= 0 does not count (:277), a
//     column none of whose values count is not a candidate; the seed mask is
//     not applied (:246-248);
//   * a candidate's total is the wrapping int32 sum of its counted scores,
//     plus trunc(gamma_bonus * scale) under HACS with gamma_bonus > 0 (:332);
//   * the CAP candidates first in (total desc, column asc) are kept (the
//     per-batch truncation of :390-393 equals a global top-CAP because columns
//     are unique per window), CAP = 32, 128 or 256 for S = roundup32(fanout)
//     <= 32, <= 128, <= 256 (macros.h DISPATCH_SAMPLING);
//   * the kept columns are sorted ascending and the first min(kept, S) are
//     the window's sample (:396-447) -- for 32 < S < CAP this is the S
//     smallest column ids of the top-CAP, not the top-S;
//   * tiles = ceil(sample / tile_cols); the output tile's slot j holds sample
//     column j (or -1) and its tile_rows values are that column's values in
//     the input window (or 0), :520-578.
//
// Design: one work-group per active window (256 threads up to 1,024 slots,
// 1,024 threads beyond, those windows' keys computed beforehand by many
// work-groups).  The 64-bit key (~total << 32 | column) orders candidates
// exactly as the reference's comparator; up to 1,024 candidates are ranked
// directly, more go through an MSB-first 8-bit radix select (passes start at
// the first byte where the candidates' keys differ) that finds the CAP-th
// key, and the selected (column, slot) pairs are compacted into LDS and
// bitonic-sorted by column.  The slot index replaces the reference's linear
// column search when the tiles are rebuilt.  Every layer of a batch can run
// in one call (grws_window_sample_layers) on device counts, with one sync.
#include "grws_internal.h"

namespace grws {
namespace {

constexpr int kBlk = 256;
constexpr int kMaxCap = 256;

enum : int32_t { kErrWindow = 1, kErrSeed = 2, kErrHacs = 4, kErrCount = 8 };

inline int bits_for(int64_t x) {
    int b = 0;
    while (b < 63 && ((int64_t)1 << b) < x) ++b;
    return b;
}

inline unsigned grid_for(int64_t n, int64_t per_block = kBlk) {
    int64_t g = (n + per_block - 1) / per_block;
    return (unsigned)(g < 1 ? 1 : g);
}

// C's (int) of a float as the GPU converts it: truncation toward zero,
// saturating at the int32 range, NaN -> 0.
__device__ __forceinline__ int32_t f2i_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}

struct ScoreParams {
    const float* static_scores;
    const int32_t* window_part_ids;
    const int32_t* part_starts;
    const int32_t* part_ends;
    int64_t num_static_scores;
    int64_t num_parts;
    float alpha, beta, delta, scale;
    int32_t gamma_int;
    int32_t use_hacs;
    int32_t locality;
};

template <typename VT>
__device__ __forceinline__ float ld_val(const void* v, int64_t i) {
    return to_float(static_cast<const VT*>(v)[i]);
}

// Key of one column slot of a window (sampling.cuh:222-345 restated per
// column): ~(total as order-preserving u32) << 32 | column, in two steps:
// slot_load reads the slot's column and its 16 values (no branch, so that
// the loads of several slots can be in flight together; every slot of a
// window's tiles has its values), slot_key_of scores them and returns false
// when the slot is not a candidate.
struct SlotRaw {
    int32_t col;
    float v[16];
};

template <typename VT>
__device__ __forceinline__ void slot_load(const int32_t* __restrict__ cols, const void* __restrict__ vals,
                                          int64_t tile0, int tc, int64_t s, SlotRaw& r) {
    const int64_t t = tile0 + s / tc;
    const int c = (int)(s % tc);
    r.col = cols[t * tc + c];
    const int64_t vbase = t * 16 * tc + c;
#pragma unroll
    for (int i = 0; i < 16; ++i) r.v[i] = ld_val<VT>(vals, vbase + (int64_t)i * tc);
}

__device__ __forceinline__ bool slot_key_of(const SlotRaw& raw, int32_t part_lo, int32_t part_hi, bool in_part_known,
                                            const ScoreParams& p, uint64_t* key) {
    // separate roundings where the reference's source writes separate
    // operations (only its 1 + 10|v| and alpha + beta|v| are fused)
#pragma clang fp contract(off)
    const int32_t col = raw.col;
    if (col == -1) return false;
    float q = 1.0f;
    bool in_part = false;
    if (p.use_hacs) {
        if (col < 0 || (int64_t)col >= p.num_static_scores) return false;  // flagged by the caller
        q = p.static_scores[col];
        in_part = in_part_known && col >= part_lo && col < part_hi;
    }
    uint32_t total = 0;
    bool any = false;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float v = fabsf(raw.v[r]);
        int32_t sc;
        if (p.use_hacs) {
            float f = __builtin_fmaf(p.beta, v, p.alpha) * q;
            if (in_part) f += p.delta;
            sc = f2i_sat(f * p.scale);
        } else {
            sc = f2i_sat(__builtin_fmaf(10.0f, v, 1.0f) * 1000.0f);
        }
        if (sc > 0) {
            total += (uint32_t)sc;
            any = true;
        }
    }
    if (!any) return false;
    total += (uint32_t)p.gamma_int;
    const uint32_t ord = total ^ 0x80000000u;  // int32 order -> u32 order
    *key = ((uint64_t)(~ord) << 32) | (uint32_t)col;
    return true;
}

template <typename VT>
__device__ __forceinline__ bool slot_key(const int32_t* __restrict__ cols, const void* __restrict__ vals,
                                         int64_t tile0, int tc, int64_t s, int32_t part_lo, int32_t part_hi,
                                         bool in_part_known, const ScoreParams& p, uint64_t* key) {
    SlotRaw r;
    slot_load<VT>(cols, vals, tile0, tc, s, r);
    return slot_key_of(r, part_lo, part_hi, in_part_known, p, key);
}

// A classify kernel lists the active windows of more than kSmallCache slots;
// two kernels share the per-window work (topk_window):
//   * window_topk_small_kernel, one 256-thread work-group per active window,
//     takes the others: a window's keys stay in LDS and are ranked directly;
//   * window_topk_big_kernel, 1,024-thread work-groups walking the list, on a
//     second stream beside it (a hub window is one long work-group): keys in
//     LDS up to kKeyCache slots, beyond that in the caller's key scratch (a
//     region claimed with one atomic on a cursor); a hub window that finds
//     the scratch full recomputes them on every pass.
// Most windows are small (c2: 10,434 of 10,584 have at most 1,024 slots),
// and at 256 threads five of them share a CU instead of two.  The radix
// passes count into one histogram per wave (a hub window's keys crowd a few
// digits).  The count
// pass also finds the least and greatest key, so the MSB-first radix select
// starts at the first byte where they differ (the bytes above are common to
// every candidate).  The count, select and compaction passes take several
// slots per thread at a time, their loads issued together.
constexpr int kTopkBlk = 1024;
constexpr int kKeyCache = 4096;
constexpr int kSmallBlk = 256;
constexpr int kSmallCache = 1024;
constexpr int kChunk = 1024;  // slots per work-group item of the keys kernel

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const uint64_t o = __shfl_xor(v, d, kWave);
        v = o < v ? o : v;
    }
    return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const uint64_t o = __shfl_xor(v, d, kWave);
        v = o > v ? o : v;
    }
    return v;
}

struct TopkArgs {
    const int64_t* win_off;
    int64_t num_windows;
    const int32_t* cols;
    const void* vals;
    int tc;
    const int32_t* active;
    int64_t num_active;             // the count, or its bound when num_active_dev is set
    const int64_t* num_active_dev;  // the count on the device (NULL: num_active)
    ScoreParams p;
    int cap;
    int S;
    int32_t* out_cols;
    int32_t* out_slots;
    int32_t* out_tiles;
    int32_t* err;
    uint64_t* gkeys;
    uint32_t* gslot;  // beside gkeys: a packed key's slot (windows of more than kKeyCache slots)
    int64_t gcap;
    unsigned long long* gcursor;
    int32_t* big_list;   // active indices of the windows left to the big kernel
    int32_t* big_count;  // their number (zero before the classify kernel)
    // per listed window i: the scratch offset of keys the keys kernel
    // computes (-1: the big kernel computes them itself), their candidate
    // count, least and greatest key, and its first chunk
    int64_t* big_goff;
    int32_t* big_cnt;
    unsigned long long* big_kmin;
    unsigned long long* big_kmax;
    int32_t* big_cbase;
    int32_t* chunk_owner;  // per chunk of kChunk slots: its window's list index, -1: none
    int32_t* chunk_total;  // chunks claimed (zero before the classify kernel)
    int64_t chunk_cap;     // chunk_owner's entries (0: no keys kernel)
};

template <int BLK, int KC, int HW>
struct TopkShared {
    int64_t goff;
    int32_t whist[HW][256];  // the radix passes' per-wave histograms
    int32_t hist[256];       // and their sum
    int32_t cnt;
    uint64_t prefix;
    int32_t shift;
    int32_t k;
    int32_t col[kMaxCap];
    int32_t slot[kMaxCap];
    uint64_t kmin[BLK / kWave], kmax[BLK / kWave];
    __attribute__((aligned(16))) uint64_t key[KC + 8];
};

// Selects active window b's sample (its columns in ascending order and their
// slots, -1 past the sample) and its output tile count.  Every thread of the
// work-group calls it with the same b; it leaves LDS to the caller's next
// window only after a barrier.
template <typename VT, int BLK, int KC, bool SMALL, int HW>
__device__ __forceinline__ void topk_window(TopkShared<BLK, KC, HW>& sh, const int64_t b, const int32_t li,
                                            const TopkArgs& a) {
    constexpr int NW = BLK / kWave;
    constexpr int FASTMAX = SMALL ? KC : BLK;  // rank directly up to this many candidates
    // slots per thread whose loads are issued together: NB in the count pass
    // (a slot's column and 16 values), NK in the select and compaction
    // passes (one key each); more do not fit the 1,024-thread kernel's 128
    // registers without spilling
    constexpr int NB = SMALL ? 1 : 2;
    constexpr int NK = SMALL ? NB : 4;
    const int tid = threadIdx.x;
    const ScoreParams& p = a.p;
    const int tc = a.tc;
    const int cap = a.cap, S = a.S;
    const int32_t w = a.active[b];
    int32_t* oc = a.out_cols + b * (int64_t)S;
    int32_t* os = a.out_slots + b * (int64_t)S;
    if (w < 0 || (int64_t)w >= a.num_windows) {
        if (tid == 0) {
            atomicOr(a.err, kErrWindow);
            a.out_tiles[b] = 0;
        }
        for (int i = tid; i < S; i += BLK) {
            oc[i] = -1;
            os[i] = -1;
        }
        return;
    }
    const int64_t t0 = a.win_off[w];
    const int64_t nslots = (a.win_off[w + 1] - t0) * tc;
    if constexpr (SMALL) {
        if (nslots > KC) return;  // listed for the big kernel
    }
    const bool cached = nslots <= KC;
    // keys the keys kernel computed (a listed window with scratch of its own)
    const int64_t pre = !SMALL && li >= 0 ? a.big_goff[li] : -1;  // uniform over the work-group
    if (tid == 0) {
        int64_t off = -1;
        if (pre >= 0) {
            off = cached ? -1 : pre;
        } else if (!cached && a.gkeys) {
            const int64_t o = (int64_t)atomicAdd(a.gcursor, (unsigned long long)nslots);
            if (o + nslots <= a.gcap) off = o;
        }
        sh.goff = off;
        sh.cnt = 0;
    }
    __syncthreads();
    uint64_t* const gk = sh.goff >= 0 ? a.gkeys + sh.goff : nullptr;  // uniform over the work-group
    int32_t part_lo = 0, part_hi = 0;
    bool in_part_known = false;
    if (p.use_hacs && p.locality && p.window_part_ids && p.part_starts && p.part_ends) {
        const int32_t pid = p.window_part_ids[w];
        if ((int64_t)pid >= p.num_parts) {
            if (tid == 0) atomicOr(a.err, kErrHacs);
        } else if (pid >= 0) {
            part_lo = p.part_starts[pid];
            part_hi = p.part_ends[pid];
            in_part_known = true;
        }
    }
    // a listed window of more than KC slots whose keys the keys kernel
    // computed holds only its items' cap smallest keys, packed, with their
    // slots beside them: the passes below scan those (nscan, set once the
    // count is known), not the window's slots
    const bool packed = !SMALL && pre >= 0 && !cached;  // uniform over the work-group
    int64_t nscan = nslots;
    // the keys of slots s + u BLK (u < NK, s + u BLK < nscan): from the LDS
    // cache or the scratch (~0: not a candidate), or recomputed
    auto keysn = [&](int64_t s, uint64_t* k, bool* c) {
        if (cached || gk) {
            const uint64_t* src = cached ? sh.key : gk;
#pragma unroll
            for (int u = 0; u < NK; ++u) {
                const int64_t su = s + (int64_t)u * BLK;
                k[u] = su < nscan ? src[su] : ~0ull;
            }
#pragma unroll
            for (int u = 0; u < NK; ++u) c[u] = k[u] != ~0ull;
        } else {  // a hub window without scratch (rare): one slot at a time
            for (int u = 0; u < NK; ++u) {
                const int64_t su = s + (int64_t)u * BLK;
                c[u] = su < nslots && slot_key<VT>(a.cols, a.vals, t0, tc, su, part_lo, part_hi, in_part_known, p, &k[u]);
            }
        }
    };

    if (pre >= 0) {
        // the keys kernel's: into LDS when they fit, else read in place
        if (cached)
            for (int64_t s = tid; s < nslots; s += BLK) sh.key[s] = a.gkeys[pre + s];
        if (tid < NW) {
            sh.kmin[tid] = a.big_kmin[li];
            sh.kmax[tid] = a.big_kmax[li];
        }
        if (tid == 0) sh.cnt = a.big_cnt[li];
    } else {
        // candidates: count, least and greatest key (and the cache)
        int local = 0;
        uint64_t kmin = ~0ull, kmax = 0;
        for (int64_t s = tid; s < nslots; s += NB * BLK) {
            SlotRaw r[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u)
                if (s + (int64_t)u * BLK < nslots) slot_load<VT>(a.cols, a.vals, t0, tc, s + (int64_t)u * BLK, r[u]);
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int64_t su = s + (int64_t)u * BLK;
                if (su >= nslots) continue;
                uint64_t k = 0;
                const bool c = slot_key_of(r[u], part_lo, part_hi, in_part_known, p, &k);
                if (cached) sh.key[su] = c ? k : ~0ull;
                else if (gk) gk[su] = c ? k : ~0ull;
                if (c) {
                    ++local;
                    kmin = k < kmin ? k : kmin;
                    kmax = k > kmax ? k : kmax;
                }
                if (p.use_hacs) {
                    const int32_t col = r[u].col;
                    if (col != -1 && (col < 0 || (int64_t)col >= p.num_static_scores)) atomicOr(a.err, kErrHacs);
                }
            }
        }
        if (local) atomicAdd(&sh.cnt, local);
        kmin = wave_min_u64(kmin);
        kmax = wave_max_u64(kmax);
        if ((tid & (kWave - 1)) == 0) {
            sh.kmin[tid / kWave] = kmin;
            sh.kmax[tid / kWave] = kmax;
        }
    }
    __syncthreads();
    const int32_t count = sh.cnt;
    if (packed) nscan = count;

    if (cached && count <= FASTMAX) {
        // a candidate's rank is the number of smaller keys (keys are
        // distinct; ~0 marks a non-candidate and is above them all), the cap
        // first are kept, and each kept one's output place is the number of
        // kept columns below its own: two passes over LDS, no select or sort.
        // Keys past nslots read as ~0: the scan runs over whole 8-key groups
        // in 16-byte LDS reads
        const int ngrp = (int)((nslots + 7) / 8);
        for (int64_t s = nslots + tid; s < 8 * (int64_t)ngrp; s += BLK) sh.key[s] = ~0ull;
        __syncthreads();
        for (int64_t s = tid; s < nslots; s += BLK) {
            const uint64_t k = sh.key[s];
            if (k == ~0ull) continue;
            int r = 0;
            const ulonglong2* kq = reinterpret_cast<const ulonglong2*>(sh.key);
            for (int g = 0; g < ngrp; ++g) {
                const ulonglong2 k0 = kq[4 * g], k1 = kq[4 * g + 1], k2 = kq[4 * g + 2], k3 = kq[4 * g + 3];
                r += (k0.x < k) + (k0.y < k) + (k1.x < k) + (k1.y < k) + (k2.x < k) + (k2.y < k) + (k3.x < k) +
                     (k3.y < k);
            }
            if (r < cap) {
                sh.col[r] = (int32_t)(uint32_t)k;
                sh.slot[r] = (int32_t)s;
            }
        }
        __syncthreads();
        const int nsel = count < cap ? count : cap;
        for (int i = tid; i < nsel; i += BLK) {
            const int32_t c = sh.col[i];
            int pos = 0;
            for (int j = 0; j < nsel; ++j) pos += sh.col[j] < c ? 1 : 0;
            if (pos < S) {
                oc[pos] = c;
                os[pos] = sh.slot[i];
            }
        }
        for (int i = nsel + tid; i < S; i += BLK) {
            oc[i] = -1;
            os[i] = -1;
        }
        const int nout = nsel < S ? nsel : S;
        if (tid == 0) a.out_tiles[b] = (nout + tc - 1) / tc;
        return;
    }
    if constexpr (!SMALL) {  // a small window always takes the direct ranking above
        static_assert(BLK >= kMaxCap, "the bitonic sort takes one thread per entry");
        // radix select of the cap-th smallest key (keys are distinct)
        uint64_t prefix = 0;
        int shift = 64;  // selected: key >> shift <= prefix >> shift (shift 64: all)
        if (count > cap) {
            uint64_t kmin = sh.kmin[0], kmax = sh.kmax[0];
#pragma unroll
            for (int i = 1; i < NW; ++i) {
                kmin = sh.kmin[i] < kmin ? sh.kmin[i] : kmin;
                kmax = sh.kmax[i] > kmax ? sh.kmax[i] : kmax;
            }
            // the bytes above the first one where the least and greatest key
            // differ are the same in every candidate
            const int hb = 63 - __clzll((long long)(kmin ^ kmax));  // count > cap >= 32: kmin != kmax
            const int sh0 = (hb / 8) * 8;
            if (tid == 0) {
                sh.k = cap;
                sh.prefix = sh0 >= 56 ? 0ull : (kmax >> (sh0 + 8)) << (sh0 + 8);
            }
            static_assert(HW == NW, "one histogram per wave");
            int32_t* const myh = sh.whist[tid / kWave];
            for (int shb = sh0; shb >= 0; shb -= 8) {
                for (int i = tid; i < NW * 256; i += BLK) sh.whist[i / 256][i % 256] = 0;
                __syncthreads();
                const uint64_t pre = sh.prefix;
                for (int64_t s = tid; s < nscan; s += NK * BLK) {
                    uint64_t k[NK];
                    bool c[NK];
                    keysn(s, k, c);
#pragma unroll
                    for (int u = 0; u < NK; ++u) {
                        if (!c[u]) continue;
                        if (shb < 56 && (k[u] >> (shb + 8)) != (pre >> (shb + 8))) continue;
                        atomicAdd(&myh[(k[u] >> shb) & 255u], 1);
                    }
                }
                __syncthreads();
                if (tid < 256) {
                    int t = 0;
#pragma unroll
                    for (int i = 0; i < NW; ++i) t += sh.whist[i][tid];
                    sh.hist[tid] = t;
                }
                __syncthreads();
                if (tid < kWave) {
                    // the first digit d whose running count reaches kk (the
                    // prefix's candidates number at least kk): lane l holds
                    // digits 4l .. 4l + 3, a wave scan finds the lane
                    const int kk = sh.k;
                    int h[4], sum = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        h[j] = sh.hist[4 * tid + j];
                        sum += h[j];
                    }
                    int incl = sum;
#pragma unroll
                    for (int dd = 1; dd < kWave; dd <<= 1) {
                        const int t = __shfl_up(incl, dd, kWave);
                        if (tid >= dd) incl += t;
                    }
                    const int excl = incl - sum;
                    if (excl < kk && kk <= incl) {
                        int below = excl, d = 4 * tid, hd = h[0];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            d = 4 * tid + j;
                            hd = h[j];
                            if (below + h[j] >= kk) break;
                            below += h[j];
                        }
                        sh.prefix = pre | ((uint64_t)d << shb);
                        sh.k = kk - below;
                        // the whole bucket is taken: no need to resolve lower digits
                        sh.shift = (below + hd == kk) ? shb : -1;
                    }
                }
                __syncthreads();
                if (sh.shift >= 0) break;
            }
            prefix = sh.prefix;
            shift = sh.shift >= 0 ? sh.shift : 0;
        }

        // compact the selected (column, slot) pairs
        if (tid == 0) sh.cnt = 0;
        for (int i = tid; i < kMaxCap; i += BLK) {
            sh.col[i] = INT32_MAX;
            sh.slot[i] = -1;
        }
        __syncthreads();
        for (int64_t s = tid; s < nscan; s += NK * BLK) {
            uint64_t k[NK];
            bool c[NK];
            keysn(s, k, c);
#pragma unroll
            for (int u = 0; u < NK; ++u) {
                if (!c[u]) continue;
                if (shift < 64 && (k[u] >> shift) > (prefix >> shift)) continue;
                const int i = atomicAdd(&sh.cnt, 1);
                if (i < kMaxCap) {
                    const int64_t su = s + (int64_t)u * BLK;
                    sh.col[i] = (int32_t)(uint32_t)k[u];
                    sh.slot[i] = packed ? (int32_t)a.gslot[sh.goff + su] : (int32_t)su;
                }
            }
        }
        __syncthreads();
        const int nsel = sh.cnt < cap ? sh.cnt : cap;

        // bitonic sort of the 256 LDS entries by column (padding INT32_MAX last)
        for (int size = 2; size <= kMaxCap; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                const int j = tid ^ stride;
                if (tid < kMaxCap && j > tid) {
                    const bool up = (tid & size) == 0;
                    const int32_t x = sh.col[tid], y = sh.col[j];
                    if ((x > y) == up) {
                        sh.col[tid] = y;
                        sh.col[j] = x;
                        const int32_t t = sh.slot[tid];
                        sh.slot[tid] = sh.slot[j];
                        sh.slot[j] = t;
                    }
                }
                __syncthreads();
            }
        }

        const int nout = nsel < S ? nsel : S;
        for (int i = tid; i < S; i += BLK) {
            oc[i] = i < nout ? sh.col[i] : -1;
            os[i] = i < nout ? sh.slot[i] : -1;
        }
        if (tid == 0) a.out_tiles[b] = (nout + tc - 1) / tc;
    }
}

// Lists the active windows of more than kSmallCache slots (in no particular
// order) for the big kernel; an invalid window id stays with the small
// kernel, which reports it.  A listed window whose keys fit the scratch and
// whose chunks fit chunk_owner gets both (its keys then come from the keys
// kernel); any other keeps big_goff -1.
__global__ __launch_bounds__(kBlk) void window_topk_classify_kernel(TopkArgs a) {
    const int64_t b = (int64_t)blockIdx.x * kBlk + threadIdx.x;
    const int64_t na = a.num_active_dev ? *a.num_active_dev : a.num_active;
    bool big = false;
    int64_t nslots = 0;
    if (b < na) {
        const int32_t w = a.active[b];
        if (w >= 0 && (int64_t)w < a.num_windows) {
            nslots = (a.win_off[w + 1] - a.win_off[w]) * a.tc;
            big = nslots > kSmallCache;
        }
    }
    const uint64_t m = __ballot(big);
    if (m == 0) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int leader = __ffsll((long long)m) - 1;
    int32_t base = 0;
    if (lane == leader) base = atomicAdd(a.big_count, __popcll(m));
    base = __shfl(base, leader, kWave);
    if (!big) return;
    const int32_t li = base + __popcll(m & lanemask_lt());
    a.big_list[li] = (int32_t)b;
    int64_t goff = -1;
    if (a.gkeys && a.chunk_cap > 0) {
        const int64_t nch = (nslots + kChunk - 1) / kChunk;
        const int64_t o = (int64_t)atomicAdd(a.gcursor, (unsigned long long)nslots);
        const int64_t cb = atomicAdd(a.chunk_total, (int32_t)nch);
        const bool ok = o + nslots <= a.gcap && cb + nch <= a.chunk_cap;
        for (int64_t j = 0; j < nch && cb + j < a.chunk_cap; ++j) a.chunk_owner[cb + j] = ok ? li : -1;
        if (ok) {
            goff = o;
            a.big_cbase[li] = (int32_t)cb;
        }
    }
    a.big_goff[li] = goff;
    a.big_cnt[li] = 0;
    a.big_kmin[li] = ~0ull;
    a.big_kmax[li] = 0ull;
}

// The listed windows' keys, kChunk slots per item, written to each window's
// scratch; every item adds its candidates to the window's count and folds
// its least and greatest key in (atomics), as the big kernel's own count
// pass would.  For a window of more than kKeyCache slots (which the big
// kernel reads in place, pass after pass) an item keeps only its cap
// smallest keys (the others cannot be among the window's cap smallest:
// keys are distinct) and packs them, with their slots, at the window's
// cursor.  Walks the chunks the classify kernel claimed; every work-group
// leaves once they are done.
static_assert(kChunk % kBlk == 0 && kChunk % 2 == 0, "whole slots per thread, key pairs in LDS");
template <typename VT>
__global__ __launch_bounds__(kBlk) void window_topk_keys_kernel(TopkArgs a) {
    constexpr int PER = kChunk / kBlk;  // slots per thread and item
    __shared__ __attribute__((aligned(16))) uint64_t skey[kChunk];
    __shared__ int scnt;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const ScoreParams& p = a.p;
    const int64_t claimed = *a.chunk_total;
    const int64_t total = claimed < a.chunk_cap ? claimed : a.chunk_cap;
    for (int64_t c = blockIdx.x; c < total; c += gridDim.x) {
        const int32_t li = a.chunk_owner[c];
        if (li < 0) continue;  // uniform over the work-group
        const int32_t w = a.active[a.big_list[li]];
        const int64_t t0 = a.win_off[w];
        const int64_t nslots = (a.win_off[w + 1] - t0) * a.tc;
        const int64_t s0 = (c - a.big_cbase[li]) * (int64_t)kChunk;
        const int64_t s1 = s0 + kChunk < nslots ? s0 + kChunk : nslots;
        uint64_t* const gk = a.gkeys + a.big_goff[li];
        uint32_t* const gs = a.gslot + a.big_goff[li];
        // windows the big kernel cannot hold in LDS get packed candidates
        const bool pack = nslots > kKeyCache;  // uniform over the work-group
        int32_t part_lo = 0, part_hi = 0;
        bool in_part_known = false;
        if (p.use_hacs && p.locality && p.window_part_ids && p.part_starts && p.part_ends) {
            const int32_t pid = p.window_part_ids[w];
            if ((int64_t)pid >= p.num_parts) {
                if (tid == 0) atomicOr(a.err, kErrHacs);
            } else if (pid >= 0) {
                part_lo = p.part_starts[pid];
                part_hi = p.part_ends[pid];
                in_part_known = true;
            }
        }
        if (tid == 0) scnt = 0;
        uint64_t kk[PER];
        int local = 0;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int64_t s = s0 + tid + u * kBlk;
            kk[u] = ~0ull;
            if (s < s1) {
                SlotRaw r;
                slot_load<VT>(a.cols, a.vals, t0, a.tc, s, r);
                uint64_t k = 0;
                if (slot_key_of(r, part_lo, part_hi, in_part_known, p, &k)) {
                    kk[u] = k;
                    ++local;
                }
                if (p.use_hacs && r.col != -1 && (r.col < 0 || (int64_t)r.col >= p.num_static_scores))
                    atomicOr(a.err, kErrHacs);
            }
            if (pack) skey[tid + u * kBlk] = kk[u];
        }
        if (pack) {
            __syncthreads();  // scnt cleared, the item's keys in LDS
            if (local) atomicAdd(&scnt, local);
            __syncthreads();
            // only the item's cap smallest keys can be among the window's cap
            // smallest (keys are distinct): the rest are dropped
            if (scnt > a.cap) {
                int rank[PER] = {};
                const ulonglong2* kq = reinterpret_cast<const ulonglong2*>(skey);
                for (int g = 0; g < kChunk / 2; ++g) {
                    const ulonglong2 q = kq[g];
#pragma unroll
                    for (int u = 0; u < PER; ++u) rank[u] += (q.x < kk[u]) + (q.y < kk[u]);
                }
#pragma unroll
                for (int u = 0; u < PER; ++u)
                    if (rank[u] >= a.cap) kk[u] = ~0ull;
            }
        }
        uint64_t kmin = ~0ull, kmax = 0;
        int kept = 0;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int64_t s = s0 + tid + u * kBlk;
            const bool keep = kk[u] != ~0ull;
            if (pack) {
                // packed at the window's cursor (its count), one atomic per wave
                const uint64_t m = __ballot(keep);
                int base = 0;
                if (lane == 0 && m) base = atomicAdd(&a.big_cnt[li], __popcll(m));
                base = __shfl(base, 0, kWave);
                if (keep) {
                    const int pos = base + __popcll(m & lanemask_lt());
                    gk[pos] = kk[u];
                    gs[pos] = (uint32_t)s;
                }
            } else if (s < s1) {
                gk[s] = kk[u];
            }
            if (keep) {
                ++kept;
                kmin = kk[u] < kmin ? kk[u] : kmin;
                kmax = kk[u] > kmax ? kk[u] : kmax;
            }
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) kept += __shfl_xor(kept, d, kWave);
        kmin = wave_min_u64(kmin);
        kmax = wave_max_u64(kmax);
        if (lane == 0 && kept > 0) {
            if (!pack) atomicAdd(&a.big_cnt[li], kept);
            atomicMin(&a.big_kmin[li], (unsigned long long)kmin);
            atomicMax(&a.big_kmax[li], (unsigned long long)kmax);
        }
        if (pack) __syncthreads();  // the LDS keys are read before the next item overwrites them
    }
}

template <typename VT>
__global__ __launch_bounds__(kSmallBlk) void window_topk_small_kernel(TopkArgs a) {
    __shared__ TopkShared<kSmallBlk, kSmallCache, 1> sh;
    const int64_t b = blockIdx.x;
    const int64_t na = a.num_active_dev ? *a.num_active_dev : a.num_active;
    if (b >= na) {  // past the device count: no tiles (the scan runs over the bound)
        if (b < a.num_active && threadIdx.x == 0) a.out_tiles[b] = 0;
        return;
    }
    topk_window<VT, kSmallBlk, kSmallCache, true, 1>(sh, b, -1, a);
}

// Walks the classify kernel's list (launched after it and after the keys
// kernel, so the count and the keys are final); every work-group leaves
// once the list is done.
template <typename VT>
__global__ __launch_bounds__(kTopkBlk) void window_topk_big_kernel(TopkArgs a) {
    __shared__ TopkShared<kTopkBlk, kKeyCache, kTopkBlk / kWave> sh;
    const int32_t n = *a.big_count;
    for (int32_t i = (int32_t)blockIdx.x; i < n; i += (int32_t)gridDim.x) {
        topk_window<VT, kTopkBlk, kKeyCache, false, kTopkBlk / kWave>(sh, a.big_list[i], i, a);
        __syncthreads();
    }
}

template <typename VT>
__global__ __launch_bounds__(kBlk) void window_recompress_kernel(const int64_t* __restrict__ win_off,
                                                                 int64_t num_windows,
                                                                 const void* __restrict__ vals, int tc,
                                                                 const int32_t* __restrict__ active,
                                                                 int64_t num_active,
                                                                 const int64_t* __restrict__ num_active_dev, int S,
                                                                 const int32_t* __restrict__ samp_cols,
                                                                 const int32_t* __restrict__ samp_slots,
                                                                 const int64_t* __restrict__ out_off,
                                                                 int32_t* __restrict__ out_cols,
                                                                 VT* __restrict__ out_vals) {
    const int64_t b = blockIdx.x;
    if (b >= (num_active_dev ? *num_active_dev : num_active)) return;
    const int64_t o0 = out_off[b];
    const int64_t ntile = out_off[b + 1] - o0;
    const int per_tile = 16 * tc;
    const int64_t total = ntile * per_tile;
    const int32_t w = active[b];
    const bool w_ok = w >= 0 && (int64_t)w < num_windows;
    const int64_t t0 = w_ok ? win_off[w] : 0;
    const int64_t nslots = w_ok ? (win_off[w + 1] - t0) * tc : 0;
    for (int64_t e = threadIdx.x; e < total; e += kBlk) {
        const int64_t t = e / per_tile;
        const int r = (int)((e % per_tile) / tc);
        const int c = (int)(e % tc);
        const int64_t j = t * tc + c;
        int32_t col = -1, slot = -1;
        if (j < S) {
            col = samp_cols[b * (int64_t)S + j];
            slot = samp_slots[b * (int64_t)S + j];
        }
        if (r == 0) out_cols[(o0 + t) * tc + c] = col;
        VT v = VT(0.0f);
        if (col != -1 && slot >= 0 && slot < nslots) {
            const int64_t it = t0 + slot / tc;
            v = static_cast<const VT*>(vals)[(it * 16 + r) * tc + slot % tc];
        }
        out_vals[(o0 + t) * per_tile + (int64_t)r * tc + c] = v;
    }
}

// --- seeds -> active windows + masks (sampling_wrapper.cu:283-347) ------
__global__ void seed_keys_kernel(const int32_t* __restrict__ ids, int64_t n, int64_t num_nodes, int tile_rows,
                                 int drop_out_of_range, uint64_t sentinel, uint64_t* __restrict__ keys,
                                 uint32_t* __restrict__ bits, int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int32_t v = ids[i];
    uint64_t k = sentinel;
    uint32_t m = 0;
    if (v >= 0 && (int64_t)v < num_nodes) {
        k = (uint64_t)(v / tile_rows);
        m = 1u << (v % tile_rows);
    } else if (v != -1 && !drop_out_of_range) {
        atomicOr(err, kErrSeed);
    }
    keys[i] = k;
    bits[i] = m;
}

__global__ void seed_heads_kernel(const uint64_t* __restrict__ keys, int64_t n, uint64_t sentinel,
                                  int32_t* __restrict__ head) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    head[i] = (keys[i] != sentinel && (i == 0 || keys[i - 1] != keys[i])) ? 1 : 0;
}

__global__ void seed_emit_kernel(const uint64_t* __restrict__ keys, const uint32_t* __restrict__ bits, int64_t n,
                                 uint64_t sentinel, const int32_t* __restrict__ head,
                                 const int64_t* __restrict__ rank, int32_t* __restrict__ windows,
                                 int32_t* __restrict__ masks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (keys[i] == sentinel) return;
    const int64_t idx = rank[i] + head[i] - 1;  // inclusive rank of this run
    if (head[i]) windows[idx] = (int32_t)keys[i];
    atomicOr(reinterpret_cast<uint32_t*>(masks) + idx, bits[i]);
}

// --- the same from a dense per-window mask (zero on entry, left zero) ----
// ids -> OR of their row bits into dense[id / 16]; n ids, or n_dev[0] * mul
// when n_dev is set (the previous layer's tiles times their columns, or an
// enqueued batch's seed count), then at most n (the bound the buffers were
// sized by; a larger device count is flagged and clamped)
__global__ __launch_bounds__(kBlk) void seeds_scatter_kernel(const int32_t* __restrict__ ids, int64_t n,
                                                             const int64_t* __restrict__ n_dev, int64_t mul,
                                                             int64_t num_nodes, int drop_out_of_range,
                                                             uint32_t* __restrict__ dense, int32_t* __restrict__ err) {
    int64_t m = n;
    if (n_dev) {
        const int64_t want = *n_dev * mul;
        if (want < 0 || want > n) {
            if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(err, kErrCount);
        } else {
            m = want;
        }
    }
    for (int64_t i = (int64_t)blockIdx.x * kBlk + threadIdx.x; i < m; i += (int64_t)gridDim.x * kBlk) {
        const int32_t v = ids[i];
        if (v >= 0 && (int64_t)v < num_nodes) atomicOr(&dense[v >> 4], 1u << (v & 15));
        else if (v != -1 && !drop_out_of_range) atomicOr(err, kErrSeed);
    }
}

__global__ __launch_bounds__(kBlk) void seeds_flags_kernel(const uint32_t* __restrict__ dense, int64_t nw,
                                                           int32_t* __restrict__ flags) {
    const int64_t w = (int64_t)blockIdx.x * kBlk + threadIdx.x;
    if (w < nw) flags[w] = dense[w] != 0u;
}

// windows in ascending order with their masks; the dense entries go back
// to zero
__global__ __launch_bounds__(kBlk) void seeds_dense_emit_kernel(uint32_t* __restrict__ dense, int64_t nw,
                                                                const int64_t* __restrict__ rank,
                                                                int32_t* __restrict__ windows,
                                                                int32_t* __restrict__ masks) {
    const int64_t w = (int64_t)blockIdx.x * kBlk + threadIdx.x;
    if (w >= nw) return;
    const uint32_t m = dense[w];
    if (m == 0u) return;
    const int64_t idx = rank[w];
    windows[idx] = (int32_t)w;
    masks[idx] = (int32_t)m;
    dense[w] = 0u;
}

// the batch's error flags beside its counts (an enqueued call's one word
// the caller reads back)
__global__ void flags_out_kernel(const int32_t* __restrict__ err, int64_t* __restrict__ out) {
    if (threadIdx.x == 0) out[0] = (int64_t)*err;
}

// a layer's active windows and tiles, kept for the one read-back at the end
__global__ void layer_counts_kernel(const int64_t* __restrict__ num_active, const int64_t* __restrict__ num_tiles,
                                    int64_t* __restrict__ out) {
    if (threadIdx.x == 0) {
        out[0] = *num_active;
        out[1] = *num_tiles;
    }
}

struct SeedWs {
    uint64_t *k, *k2;
    uint32_t *m, *m2;
    int32_t *head, *err;
    int64_t* rank;
    char* sort_ws;
    size_t sort_bytes;
    char* scan_ws;
    size_t scan_bytes;
};

template <typename C>
void carve_seed(C& cv, int64_t n, SeedWs* w) {
    const int64_t m = n > 0 ? n : 1;
    w->k = cv.template take<uint64_t>(m);
    w->k2 = cv.template take<uint64_t>(m);
    w->m = cv.template take<uint32_t>(m);
    w->m2 = cv.template take<uint32_t>(m);
    w->head = cv.template take<int32_t>(m);
    w->rank = cv.template take<int64_t>(m + 1);
    w->err = cv.template take<int32_t>(64);
    w->sort_bytes = radix_sort_workspace_bytes(m);
    w->sort_ws = cv.template take<char>(w->sort_bytes);
    w->scan_bytes = scan_workspace_bytes(m);
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

int check_graph(const grws_bcsr* A, const char* who) {
    GRWS_CHECK_ARG(A != nullptr, "%s: null graph", who);
    GRWS_CHECK_ARG(A->tile_rows == 16, "%s: tile_rows must be 16", who);
    GRWS_CHECK_ARG(A->tile_cols == 8 || A->tile_cols == 16, "%s: tile_cols must be 8 or 16", who);
    GRWS_CHECK_ARG(A->num_windows >= 0 && A->num_tiles >= 0, "%s: negative size", who);
    if (A->values_dtype != GRWS_F32 && A->values_dtype != GRWS_F16 && A->values_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "%s: unsupported values dtype %d", who, A->values_dtype);
    GRWS_CHECK_ARG(A->window_offset != nullptr, "%s: null window_offset", who);
    if (A->num_tiles > 0) GRWS_CHECK_ARG(A->col_indices && A->values, "%s: null arrays", who);
    return GRWS_OK;
}

}  // namespace
}  // namespace grws

using namespace grws;

extern "C" int32_t grws_window_sample_num(int32_t fanout) {
    if (fanout < 1) return 0;
    return ((fanout + 31) / 32) * 32;
}

extern "C" size_t grws_window_seeds_workspace_bytes(int64_t num_ids) {
    if (num_ids < 0) return 0;
    NullCarver nc;
    SeedWs w;
    carve_seed(nc, num_ids, &w);
    return nc.s.used + 256;
}

extern "C" int grws_window_seeds(const int32_t* ids, int64_t num_ids, int64_t num_nodes, int32_t tile_rows,
                                 int32_t drop_out_of_range, int32_t* active_windows, int32_t* masks,
                                 void* workspace, size_t workspace_bytes, int64_t* num_active_out, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(num_ids >= 0 && num_nodes >= 0, "window_seeds: negative size");
    GRWS_CHECK_ARG(tile_rows >= 1 && tile_rows <= 32, "window_seeds: tile_rows must be in [1, 32]");
    GRWS_CHECK_ARG(num_ids <= (int64_t)UINT32_MAX, "window_seeds: too many ids");
    GRWS_CHECK_ARG(num_active_out != nullptr, "window_seeds: null num_active_out");
    *num_active_out = 0;
    if (num_ids == 0) return GRWS_OK;
    GRWS_CHECK_ARG(ids && active_windows && masks, "window_seeds: null pointer");
    Carver cv(workspace, workspace_bytes);
    SeedWs w;
    carve_seed(cv, num_ids, &w);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "window_seeds: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const int64_t W = (num_nodes + tile_rows - 1) / tile_rows;
    const uint64_t sentinel = (uint64_t)W;
    const int bits = bits_for(W + 1);
    GRWS_TRY(fill_i32(w.err, 1, 0, stream));
    GRWS_TRY(fill_i32(masks, num_ids, 0, stream));
    hipLaunchKernelGGL(seed_keys_kernel, dim3(grid_for(num_ids)), dim3(kBlk), 0, stream, ids, num_ids, num_nodes,
                       (int)tile_rows, (int)drop_out_of_range, sentinel, w.k, w.m, w.err);
    GRWS_LAUNCH_CHECK();
    bool alt = false;
    GRWS_TRY(radix_sort_pairs(w.k, w.m, w.k2, w.m2, num_ids, bits, w.sort_ws, w.sort_bytes, stream, &alt));
    const uint64_t* k = alt ? w.k2 : w.k;
    const uint32_t* m = alt ? w.m2 : w.m;
    hipLaunchKernelGGL(seed_heads_kernel, dim3(grid_for(num_ids)), dim3(kBlk), 0, stream, k, num_ids, sentinel, w.head);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(w.head, w.rank, num_ids, false, w.scan_ws, w.scan_bytes, stream));
    hipLaunchKernelGGL(seed_emit_kernel, dim3(grid_for(num_ids)), dim3(kBlk), 0, stream, k, m, num_ids, sentinel,
                       w.head, w.rank, active_windows, masks);
    GRWS_LAUNCH_CHECK();
    int64_t na = 0;
    int32_t e = 0;
    GRWS_HIP(hipMemcpyAsync(&na, w.rank + num_ids, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&e, w.err, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    if (e & kErrSeed) return set_error(GRWS_E_RANGE, "window_seeds: a seed id is outside [0, num_nodes) and not -1");
    *num_active_out = na;
    return GRWS_OK;
}

namespace {
// topk_enqueue's fixed part of its workspace
size_t topk_fixed_bytes(int64_t num_active) {
    Sizer s;
    s.take<int32_t>((size_t)num_active + 1);  // tile counts
    s.take<int32_t>(64);                      // counters
    s.take<int32_t>((size_t)num_active + 1);  // the big kernel's list
    s.take<int64_t>((size_t)num_active + 1);  // per listed window: scratch offset,
    s.take<int32_t>((size_t)num_active + 1);  // candidate count,
    s.take<uint64_t>((size_t)num_active + 1); // least key,
    s.take<uint64_t>((size_t)num_active + 1); // greatest key,
    s.take<int32_t>((size_t)num_active + 1);  // first chunk
    s.used += scan_workspace_bytes(num_active) + 256;
    return s.used;
}
}  // namespace

extern "C" size_t grws_window_topk_workspace_bytes(int64_t num_active) {
    if (num_active < 0) return 0;
    Sizer s;
    s.take<int32_t>(64);  // the flag word
    return s.used + topk_fixed_bytes(num_active);
}

namespace {
// chunk_owner entries that cover every chunk of distinct active windows
int64_t topk_chunk_cap(const grws_bcsr* A) {
    return A->num_tiles * A->tile_cols / kChunk + A->num_windows + 1;
}
}  // namespace

// Workspace beyond grws_window_topk_workspace_bytes(num_active) is the keys
// kernel's chunk table and key scratch for the windows of more than 1,024
// slots (8 bytes per slot of each such active window).  A window whose keys
// do not fit computes them in the big kernel (into LDS up to 4,096 slots,
// recomputed on every pass beyond), with the same results.
extern "C" size_t grws_window_topk_key_scratch_bytes(const grws_bcsr* A) {
    if (!A || A->num_tiles < 0 || A->num_windows < 0) return 0;
    return align_up((size_t)topk_chunk_cap(A) * 4, 256) + (size_t)(A->num_tiles * A->tile_cols) * 8 + 512;
}

namespace grws {
namespace {

ScoreParams score_params(const grws_hacs* hacs) {
    ScoreParams p{};
    p.alpha = 1.0f;
    p.beta = 10.0f;
    p.scale = 100.0f;
    if (hacs && hacs->use_hacs) {
        p.use_hacs = 1;
        p.static_scores = hacs->static_scores;
        p.num_static_scores = hacs->num_static_scores;
        p.num_parts = hacs->num_parts;
        p.alpha = hacs->alpha;
        p.beta = hacs->beta;
        p.delta = hacs->delta;
        p.scale = hacs->score_scale;
        p.gamma_int = hacs->gamma_bonus > 0.0f ? (int32_t)(hacs->gamma_bonus * hacs->score_scale) : 0;
        p.locality = hacs->locality_enabled ? 1 : 0;
        p.window_part_ids = hacs->window_part_ids;
        p.part_starts = hacs->part_starts;
        p.part_ends = hacs->part_ends;
    }
    return p;
}

int check_hacs(const grws_bcsr* A, const grws_hacs* hacs, const char* who) {
    if (!hacs || !hacs->use_hacs) return GRWS_OK;
    GRWS_CHECK_ARG(hacs->static_scores != nullptr, "%s: HACS needs static_scores", who);
    if (hacs->locality_enabled) {
        GRWS_CHECK_ARG(hacs->window_part_ids && hacs->part_starts && hacs->part_ends,
                       "%s: locality needs window_part_ids, part_starts and part_ends", who);
        GRWS_CHECK_ARG(hacs->num_window_part_ids >= A->num_windows,
                       "%s: window_part_ids has fewer entries than the graph has windows", who);
    }
    return GRWS_OK;
}

// grws_window_topk's work without the read-back: the active windows' samples
// and the scan of their tile counts into out_window_offset (num_active + 1
// entries; with num_active_dev set, num_active is a bound, the windows past
// the device count get no tiles and every entry from there on is the
// total).  err is the caller's flag word.  workspace: at least
// grws_window_topk_workspace_bytes(num_active); the rest is the chunk table
// and key scratch.
int topk_enqueue(const grws_bcsr* A, const int32_t* active_windows, int64_t num_active,
                 const int64_t* num_active_dev, int S, const ScoreParams& p, int32_t* sampled_cols,
                 int32_t* sampled_slots, int64_t* out_window_offset, int32_t* err, void* workspace,
                 size_t workspace_bytes, hipStream_t stream, hipStream_t side_given = nullptr) {
    const int cap = S <= 32 ? 32 : (S <= 128 ? 128 : 256);
    Carver cv(workspace, workspace_bytes);
    int32_t* tiles = cv.take<int32_t>(num_active + 1);
    int32_t* ctr = cv.take<int32_t>(64);  // [0] listed windows, [1] chunks claimed, [2..3] the scratch cursor
    int32_t* big_list = cv.take<int32_t>(num_active + 1);
    int64_t* big_goff = cv.take<int64_t>(num_active + 1);
    int32_t* big_cnt = cv.take<int32_t>(num_active + 1);
    uint64_t* big_kmin = cv.take<uint64_t>(num_active + 1);
    uint64_t* big_kmax = cv.take<uint64_t>(num_active + 1);
    int32_t* big_cbase = cv.take<int32_t>(num_active + 1);
    const size_t scan_bytes = scan_workspace_bytes(num_active);
    char* scan_ws = cv.take<char>(scan_bytes);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "window_topk: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    // the rest: the chunk table and the big windows' key scratch
    uint64_t* gkeys = nullptr;
    uint32_t* gslot = nullptr;
    int64_t gcap = 0;
    int32_t* chunk_owner = nullptr;
    int64_t chunk_cap = 0;
    {
        Carver rest = cv;
        const int64_t want = topk_chunk_cap(A);
        {
            Carver probe = rest;
            int32_t* co = probe.take<int32_t>((size_t)want);
            if (probe.ok && probe.used + 256 <= probe.cap) {
                rest = probe;
                chunk_owner = co;
                chunk_cap = want;
            }
        }
        if (rest.ok && rest.used + 256 <= rest.cap) {
            const size_t left = rest.cap - rest.used - 256;
            const size_t n = left > 512 ? (left - 512) / 12 : 0;  // a key and a slot per entry
            uint64_t* keys = rest.take<uint64_t>(n);
            uint32_t* slots = rest.take<uint32_t>(n);
            if (rest.ok && n > 0) {
                gkeys = keys;
                gslot = slots;
                gcap = (int64_t)n;
            }
        }
    }
    GRWS_TRY(fill_i32(ctr, 4, 0, stream));
    TopkArgs ta{};
    ta.win_off = A->window_offset;
    ta.num_windows = A->num_windows;
    ta.cols = A->col_indices;
    ta.vals = A->values;
    ta.tc = (int)A->tile_cols;
    ta.active = active_windows;
    ta.num_active = num_active;
    ta.num_active_dev = num_active_dev;
    ta.p = p;
    ta.cap = cap;
    ta.S = S;
    ta.out_cols = sampled_cols;
    ta.out_slots = sampled_slots;
    ta.out_tiles = tiles;
    ta.err = err;
    ta.gkeys = gkeys;
    ta.gslot = gslot;
    ta.gcap = gcap;
    ta.gcursor = reinterpret_cast<unsigned long long*>(ctr + 2);
    ta.big_list = big_list;
    ta.big_count = ctr;
    ta.big_goff = big_goff;
    ta.big_cnt = big_cnt;
    ta.big_kmin = reinterpret_cast<unsigned long long*>(big_kmin);
    ta.big_kmax = reinterpret_cast<unsigned long long*>(big_kmax);
    ta.big_cbase = big_cbase;
    ta.chunk_owner = chunk_owner;
    ta.chunk_total = ctr + 1;
    ta.chunk_cap = gkeys ? chunk_cap : 0;
    // the classify kernel lists the windows of more than 1,024 slots; on the
    // side stream the keys kernel computes their keys and the big kernel
    // walks the list (at most one work-group per listed window, 1,024 at
    // most) while the small kernel takes every other window on the caller's
    // stream
    hipLaunchKernelGGL(window_topk_classify_kernel, dim3(grid_for(num_active)), dim3(kBlk), 0, stream, ta);
    GRWS_LAUNCH_CHECK();
    const unsigned big_grid = (unsigned)(num_active < 1024 ? num_active : 1024);
    constexpr unsigned kKeysGrid = 1024;  // the keys kernel's work-groups walk the chunks
    {
        SideStream ss(stream);
        GRWS_TRY(side_given ? ss.fork_to(side_given) : ss.fork());
        switch (A->values_dtype) {
            case GRWS_F32:
                hipLaunchKernelGGL(window_topk_keys_kernel<float>, dim3(kKeysGrid), dim3(kBlk), 0, ss.side, ta);
                GRWS_LAUNCH_CHECK();
                hipLaunchKernelGGL(window_topk_big_kernel<float>, dim3(big_grid), dim3(kTopkBlk), 0, ss.side, ta);
                GRWS_LAUNCH_CHECK();
                hipLaunchKernelGGL(window_topk_small_kernel<float>, dim3((unsigned)num_active), dim3(kSmallBlk), 0,
                                   stream, ta);
                break;
            case GRWS_F16:
                hipLaunchKernelGGL(window_topk_keys_kernel<_Float16>, dim3(kKeysGrid), dim3(kBlk), 0, ss.side, ta);
                GRWS_LAUNCH_CHECK();
                hipLaunchKernelGGL(window_topk_big_kernel<_Float16>, dim3(big_grid), dim3(kTopkBlk), 0, ss.side, ta);
                GRWS_LAUNCH_CHECK();
                hipLaunchKernelGGL(window_topk_small_kernel<_Float16>, dim3((unsigned)num_active), dim3(kSmallBlk), 0,
                                   stream, ta);
                break;
            default:
                hipLaunchKernelGGL(window_topk_keys_kernel<__hip_bfloat16>, dim3(kKeysGrid), dim3(kBlk), 0, ss.side,
                                   ta);
                GRWS_LAUNCH_CHECK();
                hipLaunchKernelGGL(window_topk_big_kernel<__hip_bfloat16>, dim3(big_grid), dim3(kTopkBlk), 0, ss.side,
                                   ta);
                GRWS_LAUNCH_CHECK();
                hipLaunchKernelGGL(window_topk_small_kernel<__hip_bfloat16>, dim3((unsigned)num_active),
                                   dim3(kSmallBlk), 0, stream, ta);
                break;
        }
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(ss.join());
    }
    return scan_i32_to_i64(tiles, out_window_offset, num_active, false, scan_ws, scan_bytes, stream);
}

int recompress_enqueue(const grws_bcsr* A, const int32_t* active_windows, int64_t num_active,
                       const int64_t* num_active_dev, int S, const int32_t* sampled_cols,
                       const int32_t* sampled_slots, const int64_t* out_window_offset, int32_t* out_cols,
                       void* out_values, hipStream_t stream) {
    switch (A->values_dtype) {
        case GRWS_F32:
            hipLaunchKernelGGL(window_recompress_kernel<float>, dim3((unsigned)num_active), dim3(kBlk), 0, stream,
                               A->window_offset, A->num_windows, A->values, (int)A->tile_cols, active_windows,
                               num_active, num_active_dev, S, sampled_cols, sampled_slots, out_window_offset,
                               out_cols, static_cast<float*>(out_values));
            break;
        case GRWS_F16:
            hipLaunchKernelGGL(window_recompress_kernel<_Float16>, dim3((unsigned)num_active), dim3(kBlk), 0, stream,
                               A->window_offset, A->num_windows, A->values, (int)A->tile_cols, active_windows,
                               num_active, num_active_dev, S, sampled_cols, sampled_slots, out_window_offset,
                               out_cols, static_cast<_Float16*>(out_values));
            break;
        default:
            hipLaunchKernelGGL(window_recompress_kernel<uint16_t>, dim3((unsigned)num_active), dim3(kBlk), 0, stream,
                               A->window_offset, A->num_windows, A->values, (int)A->tile_cols, active_windows,
                               num_active, num_active_dev, S, sampled_cols, sampled_slots, out_window_offset,
                               out_cols, static_cast<uint16_t*>(out_values));
            break;
    }
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

int report_topk_errors(int32_t e, const char* who) {
    if (e & kErrCount)
        return set_error(GRWS_E_CAPACITY, "%s: the seed count is above the bound the call was sized for", who);
    if (e & kErrSeed) return set_error(GRWS_E_RANGE, "%s: a seed id is outside [0, num_nodes) and not -1", who);
    if (e & kErrWindow) return set_error(GRWS_E_RANGE, "%s: an active window is outside the graph", who);
    if (e & kErrHacs) return set_error(GRWS_E_RANGE, "%s: a column has no static score or a part id has no range", who);
    return GRWS_OK;
}

}  // namespace
}  // namespace grws

extern "C" int grws_window_topk(const grws_bcsr* A, const int32_t* active_windows, int64_t num_active,
                                int32_t fanout, const grws_hacs* hacs, int32_t* sampled_cols,
                                int32_t* sampled_slots, int64_t* out_window_offset, void* workspace,
                                size_t workspace_bytes, int64_t* num_tiles_out, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_graph(A, "window_topk"));
    GRWS_CHECK_ARG(num_active >= 0, "window_topk: negative num_active");
    GRWS_CHECK_ARG(num_active <= INT32_MAX, "window_topk: too many active windows");
    GRWS_CHECK_ARG(num_tiles_out && out_window_offset, "window_topk: null output");
    const int S = grws_window_sample_num(fanout);
    GRWS_CHECK_ARG(S >= 32 && S <= kMaxCap, "window_topk: fanout must be in [1, 256] (got %d)", fanout);
    *num_tiles_out = 0;
    if (num_active == 0) return fill_i64(out_window_offset, 1, 0, stream);
    GRWS_CHECK_ARG(active_windows && sampled_cols && sampled_slots, "window_topk: null pointer");
    GRWS_TRY(check_hacs(A, hacs, "window_topk"));
    const ScoreParams p = score_params(hacs);
    // the flag word first, the rest for topk_enqueue
    Carver cv(workspace, workspace_bytes);
    int32_t* err = cv.take<int32_t>(64);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "window_topk: workspace too small");
    GRWS_TRY(fill_i32(err, 1, 0, stream));
    GRWS_TRY(topk_enqueue(A, active_windows, num_active, nullptr, S, p, sampled_cols, sampled_slots,
                          out_window_offset, err, cv.base + cv.used, cv.cap - cv.used, stream));
    int64_t T = 0;
    int32_t e = 0;
    GRWS_HIP(hipMemcpyAsync(&T, out_window_offset + num_active, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&e, err, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    GRWS_TRY(report_topk_errors(e, "window_topk"));
    *num_tiles_out = T;
    return GRWS_OK;
}

extern "C" int grws_window_recompress(const grws_bcsr* A, const int32_t* active_windows, int64_t num_active,
                                      int32_t fanout, const int32_t* sampled_cols, const int32_t* sampled_slots,
                                      const int64_t* out_window_offset, int64_t num_tiles, int32_t* out_cols,
                                      void* out_values, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_graph(A, "window_recompress"));
    GRWS_CHECK_ARG(num_active >= 0 && num_tiles >= 0, "window_recompress: negative size");
    const int S = grws_window_sample_num(fanout);
    GRWS_CHECK_ARG(S >= 32 && S <= kMaxCap, "window_recompress: fanout must be in [1, 256] (got %d)", fanout);
    if (num_active == 0 || num_tiles == 0) return GRWS_OK;
    GRWS_CHECK_ARG(active_windows && sampled_cols && sampled_slots && out_window_offset && out_cols && out_values,
                   "window_recompress: null pointer");
    switch (A->values_dtype) {
        case GRWS_F32:
            hipLaunchKernelGGL(window_recompress_kernel<float>, dim3((unsigned)num_active), dim3(kBlk), 0, stream,
                               A->window_offset, A->num_windows, A->values, (int)A->tile_cols, active_windows,
                               num_active, nullptr, S,
                               sampled_cols, sampled_slots, out_window_offset, out_cols,
                               static_cast<float*>(out_values));
            break;
        case GRWS_F16:
            hipLaunchKernelGGL(window_recompress_kernel<_Float16>, dim3((unsigned)num_active), dim3(kBlk), 0, stream,
                               A->window_offset, A->num_windows, A->values, (int)A->tile_cols, active_windows,
                               num_active, nullptr, S,
                               sampled_cols, sampled_slots, out_window_offset, out_cols,
                               static_cast<_Float16*>(out_values));
            break;
        default:
            hipLaunchKernelGGL(window_recompress_kernel<uint16_t>, dim3((unsigned)num_active), dim3(kBlk), 0, stream,
                               A->window_offset, A->num_windows, A->values, (int)A->tile_cols, active_windows,
                               num_active, nullptr, S,
                               sampled_cols, sampled_slots, out_window_offset, out_cols,
                               static_cast<uint16_t*>(out_values));
            break;
    }
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

// --- every layer in one call: sampling_wrapper.cu:365-438 with one sync ---
namespace {
struct LayerBound {
    int64_t ids;     // seed ids in (bound)
    int64_t active;  // active windows (bound)
    int64_t tiles;   // output tiles (bound)
    int S;
};

int layer_bounds(const grws_bcsr* A, int64_t num_nodes, int64_t num_seeds, const int32_t* fanouts,
                 int32_t num_layers, LayerBound* lb) {
    const int64_t nw = (num_nodes + 15) / 16;
    int64_t ids = num_seeds;
    for (int32_t l = 0; l < num_layers; ++l) {
        const int S = grws_window_sample_num(fanouts[l]);
        GRWS_CHECK_ARG(fanouts[l] >= 1 && S <= kMaxCap, "window_sample_layers: fanout must be in [1, 256] (got %d)",
                       fanouts[l]);
        lb[l].ids = ids;
        lb[l].active = ids < nw ? ids : nw;
        lb[l].tiles = lb[l].active * (S / A->tile_cols);
        lb[l].S = S;
        ids = lb[l].tiles * A->tile_cols;
    }
    return GRWS_OK;
}

constexpr int32_t kMaxLayers = 64;

template <typename C>
void carve_layers(C& cv, int64_t nw, int32_t num_layers, const LayerBound* lb, int32_t** err, int64_t** cnt,
                  uint32_t** dense, int32_t** flags, int64_t** rank, char** scan_ws, size_t* scan_bytes,
                  int32_t** scols, int32_t** sslot) {
    int64_t samp = 1;
    for (int32_t l = 0; l < num_layers; ++l) samp = lb[l].active * lb[l].S > samp ? lb[l].active * lb[l].S : samp;
    *err = cv.template take<int32_t>(64);
    *cnt = cv.template take<int64_t>(2 * (size_t)num_layers);
    *dense = cv.template take<uint32_t>((size_t)(nw > 0 ? nw : 1));
    *flags = cv.template take<int32_t>((size_t)(nw > 0 ? nw : 1));
    *rank = cv.template take<int64_t>((size_t)nw + 1);
    *scan_bytes = scan_workspace_bytes(nw > 0 ? nw : 1);
    *scan_ws = cv.template take<char>(*scan_bytes);
    *scols = cv.template take<int32_t>((size_t)samp);
    *sslot = cv.template take<int32_t>((size_t)samp);
}
}  // namespace

extern "C" int grws_window_sample_layers_bounds(const grws_bcsr* A, int64_t num_nodes, int64_t num_seeds,
                                                const int32_t* fanouts, int32_t num_layers, int64_t* max_active,
                                                int64_t* max_tiles) {
    clear_error();
    GRWS_TRY(check_graph(A, "window_sample_layers"));
    GRWS_CHECK_ARG(num_layers >= 1 && num_layers <= kMaxLayers, "window_sample_layers: 1..64 layers (got %d)",
                   num_layers);
    GRWS_CHECK_ARG(num_nodes >= 0 && num_seeds >= 0, "window_sample_layers: negative size");
    GRWS_CHECK_ARG(fanouts && max_active && max_tiles, "window_sample_layers: null pointer");
    LayerBound lb[kMaxLayers];
    GRWS_TRY(layer_bounds(A, num_nodes, num_seeds, fanouts, num_layers, lb));
    for (int32_t l = 0; l < num_layers; ++l) {
        max_active[l] = lb[l].active;
        max_tiles[l] = lb[l].tiles;
    }
    return GRWS_OK;
}

extern "C" size_t grws_window_sample_layers_workspace_bytes(const grws_bcsr* A, int64_t num_nodes,
                                                            int64_t num_seeds, const int32_t* fanouts,
                                                            int32_t num_layers) {
    if (!A || !fanouts || num_layers < 1 || num_layers > kMaxLayers || num_nodes < 0 || num_seeds < 0) return 0;
    if (A->tile_cols != 8 && A->tile_cols != 16) return 0;
    LayerBound lb[kMaxLayers];
    for (int32_t l = 0; l < num_layers; ++l)
        if (fanouts[l] < 1 || grws_window_sample_num(fanouts[l]) > kMaxCap) return 0;
    if (layer_bounds(A, num_nodes, num_seeds, fanouts, num_layers, lb) != GRWS_OK) return 0;
    NullCarver nc;
    int32_t *err, *flags, *scols, *sslot;
    int64_t *cnt, *rank;
    uint32_t* dense;
    char* scan_ws;
    size_t scan_bytes;
    carve_layers(nc, (num_nodes + 15) / 16, num_layers, lb, &err, &cnt, &dense, &flags, &rank, &scan_ws, &scan_bytes,
                 &scols, &sslot);
    size_t topk = 0;
    for (int32_t l = 0; l < num_layers; ++l) {
        const size_t t = topk_fixed_bytes(lb[l].active > 0 ? lb[l].active : 1);
        topk = t > topk ? t : topk;
    }
    return align_up(nc.s.used, 256) + topk + 256;
}

namespace {
// grws_window_sample_layers and its enqueue-only form.  Every layer's
// kernels go on `stream`.  With out_dev set (the enqueued form) the seed
// count is read on the device from num_seeds_dev[0] (num_seeds is its
// bound, the size of every buffer and grid), each layer's counts go to
// out_dev[2 l], out_dev[2 l + 1] and the error flags to out_dev[2 L], and
// nothing is synchronised or read back; otherwise the counts and flags are
// read back with one sync into counts and reported.
int window_layers(const grws_bcsr* A, int64_t num_nodes, const int32_t* seeds, int64_t num_seeds,
                  const int64_t* num_seeds_dev, const int32_t* fanouts, int32_t num_layers, const grws_hacs* hacs,
                  int64_t* const* window_offset, int32_t* const* col_indices, void* const* values,
                  int32_t* const* active_windows, int32_t* const* masks, int64_t* counts, int64_t* out_dev,
                  float* phase_ms, void* workspace, size_t workspace_bytes, hipStream_t stream,
                  hipStream_t side_given) {
    GRWS_TRY(check_graph(A, "window_sample_layers"));
    GRWS_CHECK_ARG(num_layers >= 1 && num_layers <= kMaxLayers, "window_sample_layers: 1..64 layers (got %d)",
                   num_layers);
    GRWS_CHECK_ARG(num_nodes >= 0 && num_seeds >= 0 && num_seeds <= INT32_MAX, "window_sample_layers: bad size");
    GRWS_CHECK_ARG(fanouts && window_offset && col_indices && values && active_windows && masks,
                   "window_sample_layers: null pointer");
    GRWS_CHECK_ARG(out_dev || counts, "window_sample_layers: null counts");
    GRWS_CHECK_ARG(num_seeds == 0 || seeds, "window_sample_layers: null seeds");
    GRWS_TRY(check_hacs(A, hacs, "window_sample_layers"));
    LayerBound lb[kMaxLayers];
    GRWS_TRY(layer_bounds(A, num_nodes, num_seeds, fanouts, num_layers, lb));
    for (int32_t l = 0; l < num_layers; ++l) {
        GRWS_CHECK_ARG(lb[l].active <= INT32_MAX, "window_sample_layers: too many active windows in layer %d", l);
        GRWS_CHECK_ARG(window_offset[l], "window_sample_layers: null window_offset[%d]", l);
        if (lb[l].active > 0)
            GRWS_CHECK_ARG(active_windows[l] && masks[l], "window_sample_layers: null outputs in layer %d", l);
        if (lb[l].tiles > 0)
            GRWS_CHECK_ARG(col_indices[l] && values[l], "window_sample_layers: null outputs in layer %d", l);
    }
    const bool enq = out_dev != nullptr;
    const ScoreParams p = score_params(hacs);
    const int64_t nw = (num_nodes + 15) / 16;
    Carver cv(workspace, workspace_bytes);
    int32_t *err, *flags, *scols, *sslot;
    int64_t *cnt, *rank;
    uint32_t* dense;
    char* scan_ws;
    size_t scan_bytes;
    carve_layers(cv, nw, num_layers, lb, &err, &cnt, &dense, &flags, &rank, &scan_ws, &scan_bytes, &scols, &sslot);
    if (!cv.ok)
        return set_error(GRWS_E_CAPACITY, "window_sample_layers: workspace too small (%zu < %zu)", workspace_bytes,
                         cv.used);
    char* const topk_ws = cv.base + align_up(cv.used, 256);
    const size_t topk_bytes = workspace_bytes > align_up(cv.used, 256) ? workspace_bytes - align_up(cv.used, 256) : 0;
    int64_t* const cnt_out = enq ? out_dev : cnt;  // per layer {active windows, tiles}
    GRWS_TRY(fill_i32(err, 1, 0, stream));
    GRWS_TRY(fill_i32(reinterpret_cast<int32_t*>(cnt_out), 4 * num_layers, 0, stream));
    if (nw > 0) GRWS_TRY(fill_i32(reinterpret_cast<int32_t*>(dense), nw, 0, stream));
    // phase events: before the top-K, between it and the recompression, after
    hipEvent_t ev[3 * kMaxLayers] = {};
    int nev = 0;
    struct EventGuard {
        hipEvent_t* ev;
        int* n;
        ~EventGuard() {
            for (int i = 0; i < *n; ++i) (void)hipEventDestroy(ev[i]);
        }
    } guard{ev, &nev};
    if (phase_ms && !enq) {
        for (int i = 0; i < 3 * num_layers; ++i) {
            GRWS_HIP(hipEventCreate(&ev[i]));
            nev = i + 1;
        }
    }
    const bool timed = nev > 0;
    for (int32_t l = 0; l < num_layers; ++l) {
        const LayerBound& b = lb[l];
        if (b.active == 0) {  // no seeds: an empty layer (and every later one)
            GRWS_TRY(fill_i64(window_offset[l], 1, 0, stream));
            if (timed)
                for (int k = 0; k < 3; ++k) GRWS_HIP(hipEventRecord(ev[3 * l + k], stream));
            continue;
        }
        // the layer's seeds: the batch's, else the previous layer's sampled
        // columns (-1 and columns past num_nodes dropped)
        const unsigned sgrid = (unsigned)(grid_for(b.ids) < 4096 ? grid_for(b.ids) : 4096);
        if (l == 0) {
            hipLaunchKernelGGL(seeds_scatter_kernel, dim3(sgrid), dim3(kBlk), 0, stream, seeds, num_seeds,
                               num_seeds_dev, (int64_t)1, num_nodes, 0, dense, err);
        } else {
            hipLaunchKernelGGL(seeds_scatter_kernel, dim3(sgrid), dim3(kBlk), 0, stream, col_indices[l - 1], b.ids,
                               window_offset[l - 1] + lb[l - 1].active, (int64_t)A->tile_cols, num_nodes, 1, dense,
                               err);
        }
        GRWS_LAUNCH_CHECK();
        hipLaunchKernelGGL(seeds_flags_kernel, dim3(grid_for(nw)), dim3(kBlk), 0, stream, dense, nw, flags);
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(scan_i32_to_i64(flags, rank, nw, false, scan_ws, scan_bytes, stream));
        hipLaunchKernelGGL(seeds_dense_emit_kernel, dim3(grid_for(nw)), dim3(kBlk), 0, stream, dense, nw, rank,
                           active_windows[l], masks[l]);
        GRWS_LAUNCH_CHECK();
        const int64_t* na_dev = rank + nw;
        if (timed) GRWS_HIP(hipEventRecord(ev[3 * l], stream));
        GRWS_TRY(topk_enqueue(A, active_windows[l], b.active, na_dev, b.S, p, scols, sslot, window_offset[l], err,
                              topk_ws, topk_bytes, stream, side_given));
        if (timed) GRWS_HIP(hipEventRecord(ev[3 * l + 1], stream));
        if (b.tiles > 0)
            GRWS_TRY(recompress_enqueue(A, active_windows[l], b.active, na_dev, b.S, scols, sslot, window_offset[l],
                                        col_indices[l], values[l], stream));
        if (timed) GRWS_HIP(hipEventRecord(ev[3 * l + 2], stream));
        hipLaunchKernelGGL(layer_counts_kernel, dim3(1), dim3(64), 0, stream, na_dev, window_offset[l] + b.active,
                           cnt_out + 2 * l);
        GRWS_LAUNCH_CHECK();
    }
    if (enq) {
        hipLaunchKernelGGL(flags_out_kernel, dim3(1), dim3(64), 0, stream, err, out_dev + 2 * num_layers);
        GRWS_LAUNCH_CHECK();
        return GRWS_OK;
    }
    int32_t e = 0;
    GRWS_HIP(hipMemcpyAsync(counts, cnt, sizeof(int64_t) * 2 * num_layers, hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&e, err, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    GRWS_TRY(report_topk_errors(e, "window_sample_layers"));
    if (timed) {
        for (int32_t l = 0; l < num_layers; ++l) {
            GRWS_HIP(hipEventElapsedTime(&phase_ms[2 * l], ev[3 * l], ev[3 * l + 1]));
            GRWS_HIP(hipEventElapsedTime(&phase_ms[2 * l + 1], ev[3 * l + 1], ev[3 * l + 2]));
        }
    }
    return GRWS_OK;
}
}  // namespace

extern "C" int grws_window_sample_layers(const grws_bcsr* A, int64_t num_nodes, const int32_t* seeds,
                                         int64_t num_seeds, const int32_t* fanouts, int32_t num_layers,
                                         const grws_hacs* hacs, int64_t* const* window_offset,
                                         int32_t* const* col_indices, void* const* values,
                                         int32_t* const* active_windows, int32_t* const* masks, int64_t* counts,
                                         float* phase_ms, void* workspace, size_t workspace_bytes, void* stream_) {
    clear_error();
    return window_layers(A, num_nodes, seeds, num_seeds, nullptr, fanouts, num_layers, hacs, window_offset,
                         col_indices, values, active_windows, masks, counts, nullptr, phase_ms, workspace,
                         workspace_bytes, as_stream(stream_), nullptr);
}

extern "C" int grws_window_sample_layers_enqueue(const grws_bcsr* A, int64_t num_nodes, const int32_t* seeds,
                                                 int64_t max_seeds, const int64_t* num_seeds_dev,
                                                 const int32_t* fanouts, int32_t num_layers, const grws_hacs* hacs,
                                                 int64_t* const* window_offset, int32_t* const* col_indices,
                                                 void* const* values, int32_t* const* active_windows,
                                                 int32_t* const* masks, void* workspace, size_t workspace_bytes,
                                                 int64_t* out_dev, void* stream_, void* side_stream) {
    clear_error();
    GRWS_CHECK_ARG(num_seeds_dev && out_dev, "window_sample_layers_enqueue: null device count or output");
    return window_layers(A, num_nodes, seeds, max_seeds, num_seeds_dev, fanouts, num_layers, hacs, window_offset,
                         col_indices, values, active_windows, masks, nullptr, out_dev, nullptr, workspace,
                         workspace_bytes, as_stream(stream_), static_cast<hipStream_t>(side_stream));
}

extern "C" int grws_window_sample_layers_status(int64_t err) {
    clear_error();
    return report_topk_errors((int32_t)err, "window_sample_layers");
}
