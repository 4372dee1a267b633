// BCSR row-window SpMM  Y[16W x N] = A * X  for gfx950 (MI355X).
//
// Replaces the reference's tcspmm_base_kernel (core/include/spmm_tc.cuh:40-195,
// launched by core/wrapper/spmm_wrapper.cu:33-95).  Design:
//   * one work-group per (work item, N-chunk of up to 128 columns); a work
//     item is a window or, for heavy windows, a contiguous range of its slabs
//     (16 column slots); one or two wave64s share it, splitting its slabs;
//   * the 16 X rows a slab references are gathered with 16-byte loads
//     (coalesced row segments), staged in LDS, and fed to CDNA4 MFMA:
//     v_mfma_f32_16x16x16_{f16,bf16} for 16-bit inputs (16x16x32 over slab
//     pairs for grouped tiles of 4 windows), v_mfma_f32_16x16x4_f32 for fp32;
//     fp32 accumulation in registers;
//   * a ring of register buffers keeps the next slab's gathers, A values and
//     the column indices beyond them in flight while a slab is multiplied;
//     loads are branch-free (clamped address, result masked when consumed)
//     so the wait before each slab covers that slab's loads only;
//   * A (columns, headers and values) is read with the default cache policy:
//     the streaming (non-temporal) hint was 3-5% slower on every graph
//     measured (c3 N = 608 grouped 5.56 -> 5.40 ms without it, window by
//     window 6.05 -> 5.74 ms; c4 N = 112 3.83 -> 3.70 ms);
//   * -1 padding (and any column outside [0, x_rows)) contributes zero;
//   * heavy windows are split over several items whose fp32 partial sums are
//     added in a fixed order by a second kernel: deterministic, no atomics;
//   * work-group ids are remapped so each XCD (work-groups are dealt to the 8
//     XCDs round-robin) walks a contiguous range of windows of one chunk,
//     keeping a community's X rows (one chunk wide) in that XCD's L2.
// Tuning overrides for benchmarking and tests (TuneKey below): read once
// from the environment at load, set through grws_spmm_set_tuning.
#include "grws_internal.h"

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace grws {
namespace {

// cache policy of the A-side buffer loads (column indices, tile headers and
// values): 0, the default (no streaming hint)
constexpr int kAPolicy = 0;

// Tuning overrides, for benchmarks and tests only (production calls leave
// them unset and get the measured defaults).  Each is read once from its
// environment variable when the library is loaded, and can be changed
// through grws_spmm_set_tuning; -1 means "no override".  No product call
// reads the environment.
enum TuneKey {
    kTuneNblk,     // GRWS_SPMM_NBLK: column blocks per chunk (1, 2, 4, 8, 16)
    kTuneWaves,    // GRWS_SPMM_WAVES: waves per work-group (1, 2)
    kTuneKernel,   // GRWS_SPMM_KERNEL: 1 = the element-masked kernel
    kTuneOrder,    // GRWS_SPMM_ORDER: 1 = chunk-major work order, 0 = XCD shares
    kTuneNarrow,   // GRWS_SPMM_NARROW: 1 = 128-byte gathers of 8 rows
    kTuneC320,     // GRWS_SPMM_C320: 0 = no 320-column chunks
    kTuneGrpWpw,   // GRWS_GRP_WPW: windows per wave of the grouped kernel
    kTuneGrpNblk,  // GRWS_GRP_NBLK: column blocks of the grouped kernel's first launch
    kTuneGrpC320,  // GRWS_GRP_C320: 0 = no 320-column grouped chunks
    kTuneGrpK32,   // GRWS_GRP_K32: 0 = 4-window groups on the 16x16x16 kernel, not slab pairs
    kTuneGrpDma,   // GRWS_GRP_DMA: 0 = slab pairs staged through registers, not direct loads into LDS
    kTuneCount
};
const char* const kTuneNames[kTuneCount] = {"GRWS_SPMM_NBLK",   "GRWS_SPMM_WAVES",  "GRWS_SPMM_KERNEL",
                                            "GRWS_SPMM_ORDER",  "GRWS_SPMM_NARROW", "GRWS_SPMM_C320",
                                            "GRWS_GRP_WPW",     "GRWS_GRP_NBLK",    "GRWS_GRP_C320",
                                            "GRWS_GRP_K32",     "GRWS_GRP_DMA"};
std::atomic<int> g_tune[kTuneCount];
struct TuneInit {
    TuneInit() {
        for (int i = 0; i < kTuneCount; ++i) {
            const char* e = getenv(kTuneNames[i]);
            g_tune[i].store(e ? atoi(e) : -1, std::memory_order_relaxed);
        }
    }
} g_tune_init;
inline int tune(TuneKey k) { return g_tune[k].load(std::memory_order_relaxed); }

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef int32_t i32x8_t __attribute__((ext_vector_type(8)));
typedef int32_t i32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 tr_v4f16_t;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 tr_v4bf16_t;
typedef __attribute__((address_space(3))) tr_v4f16_t lds_v4f16_t;
typedef __attribute__((address_space(3))) tr_v4bf16_t lds_v4bf16_t;
typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int XT>
struct XTraits;
template <>
struct XTraits<GRWS_F32> {
    using S = float;
    static constexpr int SZ = 4;
};
template <>
struct XTraits<GRWS_F16> {
    using S = _Float16;
    static constexpr int SZ = 2;
};
template <>
struct XTraits<GRWS_BF16> {
    using S = uint16_t;  // raw bf16 bits
    static constexpr int SZ = 2;
};

// Raw load unit for a given byte width.
template <int BYTES>
struct RawT;
template <>
struct RawT<16> { using T = u32x4_t; };
template <>
struct RawT<8> { using T = u32x2_t; };
template <>
struct RawT<4> { using T = uint32_t; };
template <>
struct RawT<2> { using T = uint16_t; };

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

struct SpmmArgs {
    const int64_t* win_off;
    const int32_t* cols;
    const void* vals;
    const int32_t* items;  // null: one item per window
    int64_t num_items;
    int64_t num_tiles;
    const void* x;
    int64_t x_rows;
    int64_t ldx;
    int64_t n_cols;
    void* y;
    int64_t ldy;
    float* partials;
    int32_t nchunks;
    uint32_t x_bytes;  // buffer path: readable bytes of x (last row: n_cols elements)
    int64_t col_base;  // first output column of chunk 0 (a launch may cover part of N)
    // packed tiles (16x16 tiles, 16-bit values): per tile 4 row groups of
    // {mask_lo, mask_hi, start}, and the nonzero values they index
    const uint32_t* hdr;
    const void* pvals;
    uint32_t pv_bytes;
    // buffer path: all XCDs walk chunk 0, then chunk 1, ... (each XCD on its
    // own window range), instead of each XCD walking its own share of the
    // (chunk, window) pairs
    int32_t chunk_major;
    // optional residual R (the y dtype): Y = A X + R on rows < res_rows
    const void* res;
    int64_t ldr;
    int64_t res_rows;
    // buffer path, 16-bit X and values, chunks of 64+ columns: gather
    // 128-byte segments of 8 rows per instruction
    int32_t narrow;
    // grouped tiles: union slabs of group q are [goff[q], goff[q+1]); the
    // group's windows are q G .. q G + G - 1 (those below num_windows)
    const int64_t* goff;
    int64_t num_windows;
};

// Output conversion for the three element types.
template <int XT>
__device__ __forceinline__ void store_out(void* y, int64_t idx, float v) {
    if constexpr (XT == GRWS_F32) {
        static_cast<float*>(y)[idx] = v;
    } else if constexpr (XT == GRWS_F16) {
        static_cast<_Float16*>(y)[idx] = (_Float16)v;
    } else {
        static_cast<uint16_t*>(y)[idx] = f32_to_bf16_bits(v);
    }
}

// Residual element as fp32 (R has the output's element type).
template <int XT>
__device__ __forceinline__ float load_res(const void* r, int64_t idx) {
    if constexpr (XT == GRWS_F32) {
        return static_cast<const float*>(r)[idx];
    } else if constexpr (XT == GRWS_F16) {
        return (float)static_cast<const _Float16*>(r)[idx];
    } else {
        return __uint_as_float((uint32_t)static_cast<const uint16_t*>(r)[idx] << 16);
    }
}

// Writes a work-group's 16 x NC result: to Y (converted, after adding the
// residual when there is one), or as an fp32 partial for a split window.
// With WPB > 1 the waves' accumulators are first added in LDS in wave order
// (deterministic); `stage_all` must hold 16 * NC floats.
template <int XT, int NBLK, int WPB, typename S>
__device__ __forceinline__ void spmm_epilogue(const SpmmArgs& a, const float4_t* acc, S* stage_all, int wave,
                                              int lane, int64_t w, int slot, int chunk, int64_t n0) {
    constexpr int NC = NBLK * 16;
    const int ag = lane >> 4;
    const int bn = lane & 15;
    const int64_t N = a.n_cols;
    // D layout of the 16x16 MFMA family: lane l, element i -> row 4*(l/16)+i, col l%16
    if constexpr (WPB > 1) {
        float* red = reinterpret_cast<float*>(stage_all);
        __syncthreads();
#pragma unroll 1
        for (int k = 0; k < WPB; ++k) {
            if (wave == k) {
#pragma unroll
                for (int b = 0; b < NBLK; ++b) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int e = (4 * ag + i) * NC + b * 16 + bn;
                        red[e] = k == 0 ? acc[b][i] : red[e] + acc[b][i];
                    }
                }
            }
            __syncthreads();
        }
        if (slot < 0) {
            const int64_t row0 = w * 16;
            for (int e = threadIdx.x; e < 16 * NC; e += 64 * WPB) {
                const int r = e / NC, c = e % NC;
                if (n0 + c < N) {
                    float v = red[e];
                    if (a.res && row0 + r < a.res_rows) v += load_res<XT>(a.res, (row0 + r) * a.ldr + n0 + c);
                    store_out<XT>(a.y, (row0 + r) * a.ldy + n0 + c, v);
                }
            }
        } else {
            float* P = a.partials + ((int64_t)slot * a.nchunks + chunk) * (16 * NC);
            for (int e = threadIdx.x; e < 16 * NC; e += 64 * WPB) P[e] = red[e];
        }
        return;
    }
    if (slot < 0) {
        const int64_t row0 = w * 16;
#pragma unroll
        for (int b = 0; b < NBLK; ++b) {
            const int64_t col = n0 + b * 16 + bn;
            if (col < N) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t row = row0 + 4 * ag + i;
                    float v = acc[b][i];
                    if (a.res && row < a.res_rows) v += load_res<XT>(a.res, row * a.ldr + col);
                    store_out<XT>(a.y, row * a.ldy + col, v);
                }
            }
        }
    } else {
        float* P = a.partials + ((int64_t)slot * a.nchunks + chunk) * (16 * NC);
#pragma unroll
        for (int b = 0; b < NBLK; ++b) {
#pragma unroll
            for (int i = 0; i < 4; ++i) P[(4 * ag + i) * NC + b * 16 + bn] = acc[b][i];
        }
    }
}

// One work-group per (work item, N-chunk); WPB waves split the item's slabs
// (wave w takes slabs sb + w, sb + w + WPB, ...) and add their partials in
// LDS in a fixed order.  Each wave runs a software pipeline over a ring of
// PF + 1 register buffers: while slab s is staged and multiplied, the X rows
// and A values of the next PF slabs are in flight, and the column indices of
// the slab after those.  Every load is unconditional (an invalid slot loads
// a clamped, valid address and its result is replaced by zero), so the
// compiler can count outstanding loads and wait only for the slab it needs.
template <int XT, bool AF32, int TC, int NBLK, bool VECT, int WPB, int PF>
__global__ __launch_bounds__(64 * WPB) void spmm_fwd_kernel(SpmmArgs a) {
    using S = typename XTraits<XT>::S;
    constexpr int SZ = XTraits<XT>::SZ;
    constexpr int NC = NBLK * 16;                  // output columns per work-group
    constexpr int VEC = VECT ? 16 / SZ : 1;        // elements per lane load
    constexpr int LDB = VEC * SZ;                  // bytes per lane load
    using LoadT = typename RawT<LDB>::T;
    constexpr int PITCH = NC + (SZ == 2 ? 8 : 4);  // LDS row pitch (elements), 16-B aligned rows
    constexpr int NLD = (16 * NC + 64 * VEC - 1) / (64 * VEC);  // lane loads per slab
    constexpr int R = PF + 1;                      // pipeline ring size
    static_assert(TC == 8 || TC == 16, "tile_cols must be 8 or 16");
    static_assert(PF >= 1 && PF <= 2, "prefetch depth 1..2");
    // the waves' stage buffers double as the fp32 reduction buffer
    static_assert(WPB == 1 || WPB * 16 * PITCH * SZ >= 16 * NC * 4, "stage too small to reduce in");

    __shared__ __attribute__((aligned(16))) S stage_all[WPB * 16 * PITCH];

    const int wave = WPB > 1 ? (int)(threadIdx.x >> 6) : 0;
    const int lane = threadIdx.x & 63;
    S* stage = stage_all + wave * (16 * PITCH);
    const int64_t total = a.num_items * a.nchunks;
    const int64_t per_xcd = (total + 7) >> 3;
    const int64_t logical = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (logical >= total) return;  // uniform over the work-group
    // chunk-major: consecutive work-groups of an XCD walk consecutive items
    // of one chunk, so a window range's X rows (one chunk wide) stay in L2
    const int64_t item = logical % a.num_items;
    const int chunk = (int)(logical / a.num_items);
    const int64_t col_base = a.col_base;

    int64_t w, sb, se;
    int slot;
    if (a.items) {
        const int32_t* it = a.items + 4 * item;
        w = it[0];
        sb = it[1];
        se = it[2];
        slot = it[3];
    } else {
        w = item;
        sb = 0;
        se = INT64_MAX;
        slot = -1;
    }
    int64_t t1 = a.win_off[w + 1];
    int64_t t0 = a.win_off[w];
    // malformed offsets must never read outside the tile arrays
    t1 = t1 < 0 ? 0 : (t1 > a.num_tiles ? a.num_tiles : t1);
    t0 = t0 < 0 ? 0 : (t0 > t1 ? t1 : t0);
    const int64_t nslots = (t1 - t0) * TC;
    const int64_t nslabs = (nslots + 15) >> 4;
    if (se > nslabs) se = nslabs;
    if (sb > se) sb = se;

    const int64_t n0 = col_base + (int64_t)chunk * NC;
    const int64_t N = a.n_cols;
    const uint32_t xr = (uint32_t)a.x_rows;
    const S* __restrict__ X = static_cast<const S*>(a.x);
    const int32_t* __restrict__ colp = a.cols + t0 * TC;

    // per-lane load geometry (compile-time per lane position)
    int ld_row[NLD], ld_col[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        int e = (i * 64 + lane) * VEC;
        ld_row[i] = e / NC;
        ld_col[i] = e % NC;
    }

    // A (column indices and values) is read once per chunk
    auto load_cols = [&](int64_t s) -> int {
        const int64_t sl = s * 16 + (lane & 15);
        const bool ok = s < se && sl < nslots;
        const int v = colp[ok ? sl : 0];
        return ok ? v : -1;
    };
    // Returns the validity bits of the NLD loads; invalid lanes load a
    // clamped address and are zeroed only when the slab is consumed, so no
    // select waits on a load that was just issued.
    auto load_x = [&](int cv, LoadT* regs) -> uint32_t {
        uint32_t okm = 0;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int r = ld_row[i];
            const int c = __shfl(cv, r & 15, 64);
            const bool ok = (r < 16) && ((uint32_t)c < xr) && (n0 + ld_col[i] < N);
            regs[i] = *reinterpret_cast<const LoadT*>(X + (ok ? (int64_t)c * a.ldx + n0 + ld_col[i] : 0));
            okm |= (ok ? 1u : 0u) << i;
        }
        return okm;
    };

    // A fragment: row r = lane%16, slots 16s + 4g .. 16s + 4g + 3 (g = lane/16)
    const int ar = lane & 15;
    const int ag = lane >> 4;
    using AVec = typename std::conditional<AF32, float4_t, typename std::conditional<XT == GRWS_F32, float4_t, u32x2_t>::type>::type;
    // the A fragment of an invalid slab is zeroed at consumption as well
    auto a_valid = [&](int64_t s) -> bool { return s < se && s * 16 + 4 * ag < nslots; };
    auto load_a = [&](int64_t s) -> AVec {
        const int64_t sl = s * 16 + 4 * ag;
        const bool ok = s < se && sl < nslots;
        const int64_t slc = ok ? sl : 0;
        const int64_t off = ok ? ((t0 + slc / TC) * 16 + ar) * TC + (slc % TC) : 0;
        if constexpr (AF32 || XT == GRWS_F32) {
            return *reinterpret_cast<const float4_t*>(static_cast<const float*>(a.vals) + off);
        } else {
            return *reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(a.vals) + off);
        }
    };

    float4_t acc[NBLK];
#pragma unroll
    for (int b = 0; b < NBLK; ++b) acc[b] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int bn = lane & 15;
    auto consume = [&](const LoadT* xb, const uint32_t okm, const AVec a_raw, const bool a_ok) {
        const AVec a_cur = a_ok ? a_raw : AVec{};
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            if (ld_row[i] < 16)
                *reinterpret_cast<LoadT*>(&stage[ld_row[i] * PITCH + ld_col[i]]) = ((okm >> i) & 1u) ? xb[i] : LoadT{};
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if constexpr (XT == GRWS_F32) {
            float4_t af = a_cur;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int k = 4 * ag + q;
#pragma unroll
                for (int b = 0; b < NBLK; ++b) {
                    float bv = stage[k * PITCH + b * 16 + bn];
                    acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[q], bv, acc[b], 0, 0, 0);
                }
            }
        } else if constexpr (XT == GRWS_F16) {
            half4_t af;
            if constexpr (AF32) {
                af = half4_t{(_Float16)a_cur[0], (_Float16)a_cur[1], (_Float16)a_cur[2], (_Float16)a_cur[3]};
            } else {
                af = __builtin_bit_cast(half4_t, a_cur);
            }
#pragma unroll
            for (int b = 0; b < NBLK; ++b) {
                const S* p = stage + (4 * ag) * PITCH + b * 16 + bn;
                half4_t bf = half4_t{p[0], p[PITCH], p[2 * PITCH], p[3 * PITCH]};
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(af, bf, acc[b], 0, 0, 0);
            }
        } else {
            short4_t af;
            if constexpr (AF32) {
                af = short4_t{(short)f32_to_bf16_bits(a_cur[0]), (short)f32_to_bf16_bits(a_cur[1]),
                              (short)f32_to_bf16_bits(a_cur[2]), (short)f32_to_bf16_bits(a_cur[3])};
            } else {
                af = __builtin_bit_cast(short4_t, a_cur);
            }
#pragma unroll
            for (int b = 0; b < NBLK; ++b) {
                const S* p = stage + (4 * ag) * PITCH + b * 16 + bn;
                short4_t bf = short4_t{(short)p[0], (short)p[PITCH], (short)p[2 * PITCH], (short)p[3 * PITCH]};
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(af, bf, acc[b], 0, 0, 0);
            }
        }
        // the next slab overwrites the stage
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    const int64_t s0 = sb + wave;
    if (s0 < se && xr > 0) {  // uniform per wave; every load below is in bounds
        LoadT buf[R][NLD];
        AVec abuf[R];
        uint32_t okx[R];
        int cring[R];
#pragma unroll
        for (int k = 0; k < R; ++k) cring[k] = load_cols(s0 + (int64_t)k * WPB);
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            okx[k] = load_x(cring[k], buf[k]);
            abuf[k] = load_a(s0 + (int64_t)k * WPB);
        }
        // one pipeline step for slab s in ring slot u
        auto step = [&](const int u, const int64_t s) {
            const int ps = (u + PF) % R;  // ring slot of slab s + PF*WPB
            // columns of slab s + R*WPB into the slot slab s no longer needs
            cring[u] = load_cols(s + (int64_t)R * WPB);
            okx[ps] = load_x(cring[ps], buf[ps]);
            abuf[ps] = load_a(s + (int64_t)PF * WPB);
            consume(buf[u], okx[u], abuf[u], a_valid(s));
        };
        // whole ring turns without exits (uniform load counts), then the rest
        const int64_t nsteps = (se - s0 + WPB - 1) / WPB;
        const int64_t nturns = nsteps / R;
        int64_t s = s0;
        for (int64_t t = 0; t < nturns; ++t) {
#pragma unroll
            for (int u = 0; u < R; ++u) {
                step(u, s);
                s += WPB;
            }
        }
        const int rest = (int)(nsteps - nturns * R);
#pragma unroll
        for (int u = 0; u < R - 1; ++u) {
            if (u < rest) step(u, s);
            s += WPB;
        }
    }

    spmm_epilogue<XT, NBLK, WPB>(a, acc, stage_all, wave, lane, w, slot, chunk, n0);
}

// Buffer-load variant for 16-bit X (the common case).  Same work mapping,
// ring pipeline and arithmetic as spmm_fwd_kernel, with the per-slab
// instruction count cut down:
//   * X, A and the column indices are read with raw buffer loads whose
//     range check returns zero past the end of the resource: an invalid
//     column is redirected to row x_rows (out of range), A and the column
//     indices use one resource per work item, so no load needs a mask or a
//     select when consumed and row offsets are 32-bit (24 x 24 multiply);
//   * lane l gathers NLD consecutive rows of the slab, so its column
//     indices come from one vector load instead of cross-lane shuffles;
//   * the B operand of each MFMA is one ds_read_b64_tr_b16 (gfx950's LDS
//     transpose read): lane k of each 16-lane group reads 4 halves of stage
//     row 4*(l/16) + k/4 at column 16*b + 4*(k%4), and the group's 64 halves
//     come back transposed so lane i holds column i of rows 4g..4g+3.
// Requires (checked on the host): x_rows < 2^24, row pitch < 2^24 bytes,
// x_rows + 1 rows of X addressable in 32 bits, and every work item's
// A within 2^31 bytes.
//
// PK: A comes from packed tiles instead of the dense 16x16 values.  A tile's
// 256 slots (row-major) form 4 groups of 4 rows; group q has a 64-bit mask
// (bit (r%4)*16 + c set iff slot (r, c) holds a value whose bits are not
// zero) and the index of its first value in the packed array, where the
// nonzero values follow in slot order.  Lane (ag, ar) needs slots
// ar*16 + 4ag .. +3: its mask nibble, and the popcount of the mask bits
// below it added to the group start locate its values; a 12-byte load and
// a byte permute rebuild the 4 halves with zeros in the empty slots, so
// the MFMA sees exactly the dense tile's operand (bit-identical results).
// The header rides in the column-index ring, loaded a step before the
// dependent value read, which so adds no wait of its own.
template <int XT, bool AF32, int TC, int NBLK, int WPB, int PF, bool PK = false, bool NR = false>
__global__ __launch_bounds__(64 * WPB) __attribute__((amdgpu_waves_per_eu(NBLK == 20 ? 3 : 1, 8))) void spmm_buf_kernel(
    SpmmArgs a) {
    static_assert(XT == GRWS_F16 || XT == GRWS_BF16 || (XT == GRWS_F32 && AF32 && !PK),
                  "16-bit X, or fp32 X with fp32 values");
    static_assert(TC == 8 || TC == 16, "tile_cols must be 8 or 16");
    static_assert(PF >= 1 && PF <= 2, "prefetch depth 1..2");
    static_assert(!PK || (TC == 16 && !AF32), "packed tiles: 16x16 tiles of 16-bit values");
    using S = typename XTraits<XT>::S;
    constexpr bool XF32 = XT == GRWS_F32;
    constexpr int SZ = XTraits<XT>::SZ;
    constexpr int SZA = AF32 ? 4 : 2;
    constexpr int NC = NBLK * 16;               // output columns per work-group
    constexpr int VEC = 16 / SZ;                // elements per 16-byte load
    constexpr int LPR = NC / VEC;               // lanes per staged row
    constexpr int NLD = (16 * LPR + 63) / 64;   // rows (loads) per lane per slab
    // LDS row pitch (elements).  fp32: the 4 k-groups of a B read (rows
    // 4g + q, g = 0..3) then start 16 banks apart (no conflict)
    constexpr int PITCH = XF32 ? NC + 4 : NC + 16;
    static_assert(NR || NLD == 1 || NLD == 2 || NLD == 4 || NLD == 8, "rows per lane");
    // NR: every gather instruction reads 128-byte segments of 8 slab rows (8
    // lanes per segment) instead of NC*SZ-byte runs of 64/LPR rows; the same
    // NLD loads per lane, each lane on 2 rows (rsub, 8 + rsub)
    static_assert(!NR || (!XF32 && NC % 64 == 0), "narrow segments: 16-bit X, NC a multiple of 64");
    constexpr int SEGS = NR ? NC / 64 : 1;  // 128-byte segments per staged row
    constexpr int R = PF + 1;
    static_assert(WPB == 1 || WPB * 16 * PITCH * SZ >= 16 * NC * 4, "stage too small to reduce in");
    using ColV = typename std::conditional<
        NR, i32x2_t,
        typename std::conditional<
            NLD == 8, i32x8_t,
            typename std::conditional<NLD == 4, i32x4_t,
                                      typename std::conditional<NLD == 2, i32x2_t, int32_t>::type>::type>::type>::type;
    using AVec = typename std::conditional<PK, u32x4_t,
                                           typename std::conditional<AF32, float4_t, u32x2_t>::type>::type;
    using HdrV = typename std::conditional<PK, u32x3_t, int>::type;

    __shared__ __attribute__((aligned(16))) S stage_all[WPB * 16 * PITCH];

    const int wave = WPB > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;
    const int lane = threadIdx.x & 63;
    S* stage = stage_all + wave * (16 * PITCH);
    int64_t item;
    int chunk;
    if (a.chunk_major) {
        const int64_t ipc = (a.num_items + 7) & ~(int64_t)7;  // work-groups per chunk
        chunk = (int)(blockIdx.x / ipc);
        const int64_t r = (int64_t)blockIdx.x - (int64_t)chunk * ipc;
        item = (r & 7) * (ipc >> 3) + (r >> 3);
        if (chunk >= a.nchunks || item >= a.num_items) return;  // uniform over the work-group
    } else {
        const int64_t total = a.num_items * a.nchunks;
        const int64_t per_xcd = (total + 7) >> 3;
        const int64_t logical = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
        if (logical >= total) return;  // uniform over the work-group
        item = logical % a.num_items;
        chunk = (int)(logical / a.num_items);
    }
    const int64_t col_base = a.col_base;

    int64_t w, sb, se;
    int slot;
    if (a.items) {
        const int32_t* it = a.items + 4 * item;
        w = it[0];
        sb = it[1];
        se = it[2];
        slot = it[3];
    } else {
        w = item;
        sb = 0;
        se = INT64_MAX;
        slot = -1;
    }
    int64_t t1 = a.win_off[w + 1];
    int64_t t0 = a.win_off[w];
    t1 = t1 < 0 ? 0 : (t1 > a.num_tiles ? a.num_tiles : t1);
    t0 = t0 < 0 ? 0 : (t0 > t1 ? t1 : t0);
    const int64_t nslots = (t1 - t0) * TC;
    const int64_t nslabs = (nslots + 15) >> 4;
    if (se > nslabs) se = nslabs;
    if (sb > se) sb = se;
    const int64_t n0 = col_base + (int64_t)chunk * NC;

    // one resource per work item for A and the column indices, starting at
    // slab sb; reads beyond the window return zero
    const int64_t a_bytes = nslots * 16 * SZA - sb * 256 * SZA;
    const int64_t c_bytes = (nslots - sb * 16) * 4;
    const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const char*>(a.vals) + (t0 * 16 * TC + sb * 256) * SZA), (short)0,
        (int)(a_bytes > 0x7fffffff ? 0x7fffffff : (a_bytes < 0 ? 0 : a_bytes)), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsC = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.cols + t0 * TC + sb * 16), (short)0, (int)(c_bytes < 0 ? 0 : c_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsX =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.x), (short)0, (int)a.x_bytes, 0x00020000);
    // packed tiles: headers of the item's tiles from slab sb (slab = tile at
    // tile_cols 16), and all packed values; reads past either return zero
    auto make_h = [&]() {
        if constexpr (PK) {
            const int64_t h_bytes = (nslabs - sb) * 48;
            return __builtin_amdgcn_make_buffer_rsrc((void*)(a.hdr + (t0 + sb) * 12), (short)0,
                                                     (int)(h_bytes > 0x7fffffff ? 0x7fffffff : h_bytes), 0x00020000);
        } else {
            return __builtin_amdgcn_make_buffer_rsrc(nullptr, (short)0, 0, 0x00020000);
        }
    };
    const __amdgpu_buffer_rsrc_t rsH = make_h();
    const __amdgpu_buffer_rsrc_t rsV = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(PK ? a.pvals : nullptr),
                                                                         (short)0, PK ? (int)a.pv_bytes : 0, 0x00020000);

    const int rbase = NR ? (lane >> 3) : NLD * (lane / LPR);  // the lane's first slab row
    const bool lrow = NR || rbase < 16;   // NBLK == 1: lanes 32..63 stage nothing
    // a lane whose columns lie past n_cols (the last chunk) reads nothing:
    // it always takes row x_rows, which lies past the resource (so every
    // offset stays below (x_rows + 1) rows).  Column element of load i:
    // (lane % LPR) * VEC, or with NR 64 (i % SEGS) + 8 (lane % 8)
    int lce[SEGS];
    bool lcol[SEGS];
    uint32_t colb[SEGS];
#pragma unroll
    for (int g = 0; g < SEGS; ++g) {
        lce[g] = NR ? 64 * g + 8 * (lane & 7) : (lane % LPR) * VEC;
        lcol[g] = n0 + lce[g] < a.n_cols;
        colb[g] = lcol[g] ? (uint32_t)((n0 + lce[g]) * SZ) : 0u;
    }
    // slab row of the lane's load i
    auto row_of = [&](int i) { return NR ? 8 * (i / SEGS) + rbase : rbase + i; };
    const uint32_t ldxb = (uint32_t)(a.ldx * SZ);
    const uint32_t xr = (uint32_t)a.x_rows;
    const int ag = lane >> 4;
    const int ar = lane & 15;
    // A fragment: row ar, slots 4ag..4ag+3 of the slab (values are [tile][row][col])
    const uint32_t a_lane = (uint32_t)((((4 * ag) / TC) * 16 + ar) * TC + (4 * ag) % TC) * SZA;
    // transpose-read address of this lane within a 16-column block
    const int tr_off = (4 * ag + ((lane & 15) >> 2)) * PITCH + 4 * (lane & 3);
    // packed tiles: this lane's row group header and its first mask bit
    const uint32_t h_lane = (uint32_t)(ar >> 2) * 12;
    const uint32_t bitoff = (uint32_t)((ar & 3) * 16 + 4 * ag);

    auto load_cols = [&](int64_t s) -> ColV {
        const uint32_t off = (uint32_t)((s - sb) * 64) + (uint32_t)rbase * 4;
        if constexpr (NR) {
            return ColV{(int32_t)__builtin_amdgcn_raw_buffer_load_b32(rsC, (int)off, 0, kAPolicy),
                        (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rsC, (int)(off + 32), 0, kAPolicy)};
        } else if constexpr (NLD == 8) {
            const u32x4_t lo = __builtin_amdgcn_raw_buffer_load_b128(rsC, (int)off, 0, kAPolicy);
            const u32x4_t hi = __builtin_amdgcn_raw_buffer_load_b128(rsC, (int)(off + 16), 0, kAPolicy);
            return ColV{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        } else if constexpr (NLD == 4) {
            return __builtin_bit_cast(ColV, __builtin_amdgcn_raw_buffer_load_b128(rsC, (int)off, 0, kAPolicy));
        } else if constexpr (NLD == 2) {
            return __builtin_bit_cast(ColV, __builtin_amdgcn_raw_buffer_load_b64(rsC, (int)off, 0, kAPolicy));
        } else {
            return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rsC, (int)off, 0, kAPolicy);
        }
    };
    auto load_x = [&](const ColV cv, int64_t s, u32x4_t* regs) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            int32_t c;
            if constexpr (NR) c = cv[i / SEGS]; else if constexpr (NLD == 1) c = cv; else c = cv[i];
            bool ok = lrow && lcol[i % SEGS] && (uint32_t)c < xr;
            if constexpr (TC == 8) ok = ok && (s * 16 + row_of(i) < nslots);  // half-empty last slab
            const uint32_t row = ok ? (uint32_t)c : xr;  // row x_rows lies past the resource
            regs[i] = __builtin_amdgcn_raw_buffer_load_b128(rsX, (int)(__umul24(row, ldxb) + colb[i % SEGS]), 0, 0);
        }
    };
    auto load_hdr = [&](int64_t s) -> HdrV {
        if constexpr (PK) {
            return __builtin_amdgcn_raw_buffer_load_b96(rsH, (int)((uint32_t)((s - sb) * 48) + h_lane), 0, kAPolicy);
        } else {
            return 0;
        }
    };
    auto load_a = [&](int64_t s, const HdrV h) -> AVec {
        if constexpr (PK) {
            // {d0, d1, d2} hold the lane's run of up to 4 values starting
            // at the low half of d0, or at its high half when info bit 4 is set
            const uint64_t m = ((uint64_t)h[1] << 32) | h[0];
            const uint32_t below = (uint32_t)__builtin_popcountll(m & ((1ull << bitoff) - 1));
            const uint32_t nib = (uint32_t)(m >> bitoff) & 15u;
            const uint32_t hidx = h[2] + below;
            const uint32_t off = nib ? (hidx & ~1u) * 2u : 0x80000000u;  // empty: no read
            const u32x3_t d = __builtin_amdgcn_raw_buffer_load_b96(rsV, (int)off, 0, kAPolicy);
            return u32x4_t{d[0], d[1], d[2], nib | ((hidx & 1u) << 4)};
        } else {
            (void)h;
            const uint32_t off = (uint32_t)((s - sb) * 256 * SZA) + a_lane;
            if constexpr (AF32) {
                return __builtin_bit_cast(AVec, __builtin_amdgcn_raw_buffer_load_b128(rsA, (int)off, 0, kAPolicy));
            } else {
                return __builtin_bit_cast(AVec, __builtin_amdgcn_raw_buffer_load_b64(rsA, (int)off, 0, kAPolicy));
            }
        }
    };

    float4_t acc[NBLK];
#pragma unroll
    for (int b = 0; b < NBLK; ++b) acc[b] = float4_t{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](const u32x4_t* xb, const AVec a_cur) {
        if (lrow) {
#pragma unroll
            for (int i = 0; i < NLD; ++i)
                *reinterpret_cast<u32x4_t*>(&stage[row_of(i) * PITCH + lce[i % SEGS]]) = xb[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if constexpr (XF32) {
            // v_mfma_f32_16x16x4f32: lane (ag, ar) holds A[ar][4ag + q] for the
            // q-th of 4 MFMAs, and reads B[4ag + q][16b + ar] from the stage
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
                for (int b = 0; b < NBLK; ++b) {
                    const float bv = stage[(4 * ag + q) * PITCH + b * 16 + ar];
                    acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a_cur[q], bv, acc[b], 0, 0, 0);
                }
            }
        } else {
        short4_t af;
        if constexpr (PK) {
            const uint32_t info = a_cur[3];
            const uint32_t sh = (info >> 4) * 16u;
            const uint32_t r0 = __builtin_amdgcn_alignbit(a_cur[1], a_cur[0], sh);
            const uint32_t r1 = __builtin_amdgcn_alignbit(a_cur[2], a_cur[1], sh);
            // selector of slot j: bytes of run value rank_j, or 0x0c (zero byte)
            const uint32_t b0 = info & 1u, b1 = (info >> 1) & 1u, b2 = (info >> 2) & 1u, b3 = (info >> 3) & 1u;
            const uint32_t k2 = b0 + b1, k3 = k2 + b2;
            const uint32_t s0 = b0 ? 0x0100u : 0x0c0cu;
            const uint32_t s1 = b1 ? 0x0100u + 0x0202u * b0 : 0x0c0cu;
            const uint32_t s2 = b2 ? 0x0100u + 0x0202u * k2 : 0x0c0cu;
            const uint32_t s3 = b3 ? 0x0100u + 0x0202u * k3 : 0x0c0cu;
            af = __builtin_bit_cast(short4_t, u32x2_t{__builtin_amdgcn_perm(r1, r0, s0 | (s1 << 16)),
                                                      __builtin_amdgcn_perm(r1, r0, s2 | (s3 << 16))});
        } else if constexpr (AF32) {
            if constexpr (XT == GRWS_F16) {
                af = __builtin_bit_cast(short4_t, half4_t{(_Float16)a_cur[0], (_Float16)a_cur[1], (_Float16)a_cur[2],
                                                          (_Float16)a_cur[3]});
            } else {
                af = short4_t{(short)f32_to_bf16_bits(a_cur[0]), (short)f32_to_bf16_bits(a_cur[1]),
                              (short)f32_to_bf16_bits(a_cur[2]), (short)f32_to_bf16_bits(a_cur[3])};
            }
        } else {
            af = __builtin_bit_cast(short4_t, a_cur);
        }
#pragma unroll
        for (int b = 0; b < NBLK; ++b) {
            lds_ptr_t p = (lds_ptr_t)(stage + tr_off + 16 * b);
            if constexpr (XT == GRWS_F16) {
                const half4_t bf = __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                                                   (lds_v4f16_t*)p));
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, af), bf, acc[b], 0, 0, 0);
            } else {
                const short4_t bf = __builtin_bit_cast(short4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                                                                     (lds_v4bf16_t*)p));
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(af, bf, acc[b], 0, 0, 0);
            }
        }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    const int64_t s0 = sb + wave;
    if (s0 < se && xr > 0) {  // uniform per wave
        // Ring of R = PF + 1 slots: each step issues the column indices R
        // slabs ahead (and, for packed tiles, their headers), the X rows and
        // A values PF slabs ahead, then multiplies the current slab.
        u32x4_t buf[R][NLD];
        AVec abuf[R];
        ColV cring[R];
        HdrV hring[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            cring[k] = load_cols(s0 + (int64_t)k * WPB);
            hring[k] = load_hdr(s0 + (int64_t)k * WPB);
        }
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            load_x(cring[k], s0 + (int64_t)k * WPB, buf[k]);
            abuf[k] = load_a(s0 + (int64_t)k * WPB, hring[k]);
        }
        auto step = [&](const int u, const int64_t s) {
            const int ps = (u + PF) % R;
            cring[u] = load_cols(s + (int64_t)R * WPB);
            hring[u] = load_hdr(s + (int64_t)R * WPB);
            load_x(cring[ps], s + (int64_t)PF * WPB, buf[ps]);
            abuf[ps] = load_a(s + (int64_t)PF * WPB, hring[ps]);
            consume(buf[u], abuf[u]);
        };
        const int64_t nsteps = (se - s0 + WPB - 1) / WPB;
        const int64_t nturns = nsteps / R;
        int64_t s = s0;
        for (int64_t t = 0; t < nturns; ++t) {
#pragma unroll
            for (int u = 0; u < R; ++u) {
                step(u, s);
                s += WPB;
            }
        }
        const int rest = (int)(nsteps - nturns * R);
#pragma unroll
        for (int u = 0; u < R - 1; ++u) {
            if (u < rest) step(u, s);
            s += WPB;
        }
    }
    spmm_epilogue<XT, NBLK, WPB>(a, acc, stage_all, wave, lane, w, slot, chunk, n0);
}

// Grouped tiles (group.hip builds them): G consecutive windows share one
// sorted list of their columns in slabs of 16 and keep one packed 16x16
// sub-tile each per slab (same packing as PK above).  A work-group of GW
// waves takes one group and one N-chunk; each wave owns WPW of the group's
// windows (G = WPW GW).  Per slab the waves gather the slab's 16 X rows
// once, wave h the rows [h 16/GW, (h+1) 16/GW) in 128-byte segments, 8
// per instruction (a last partial instruction repeats segments of the same
// rows: its extra lanes write what other lanes write), into LDS; then every
// wave multiplies each staged 16-column block by its windows' sub-tiles,
// one transposing LDS read serving WPW MFMAs.  With GW > 1 the stage is double buffered and one
// barrier per slab orders its writes before its reads (a buffer is written
// again two slabs later, after every wave passed the barrier in between).
template <int XT, int NBLK, int WPW, int GW, int PF>
__global__ __launch_bounds__(64 * GW) void spmm_grp_kernel(SpmmArgs a) {
    static_assert(XT == GRWS_F16 || XT == GRWS_BF16, "grouped tiles: 16-bit X and values");
    static_assert(GW == 1 || GW == 2 || GW == 4, "waves per group");
    static_assert(PF >= 1 && PF <= 2, "prefetch depth 1..2");
    constexpr int G = WPW * GW;
    constexpr int NC = NBLK * 16;
    constexpr int SEGS = NC / 64;       // 128-byte segments per staged row
    constexpr int RPW = 16 / GW;        // staged rows each wave gathers
    constexpr int NSEG = RPW * SEGS;
    constexpr int NLD = (NSEG + 7) / 8; // gather instructions per wave and slab
    constexpr int PAD = NLD * 8 - NSEG;
    static_assert(NC % 64 == 0 && PAD % RPW == 0 && PAD < 8, "gather instructions per wave");
    constexpr int PITCH = NC + 16;
    constexpr int NST = GW > 1 ? 2 : 1;
    constexpr int R = PF + 1;
    using S = typename XTraits<XT>::S;
    using ColV = typename std::conditional<GW == 1, i32x2_t, int32_t>::type;
    __shared__ __attribute__((aligned(16))) S stage_all[NST * 16 * PITCH];

    const int wave = GW > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;
    const int lane = threadIdx.x & 63;
    // chunk-major: every XCD walks chunk 0's groups (its own range), then chunk 1's
    const int64_t ipc = (a.num_items + 7) & ~(int64_t)7;
    const int chunk = (int)(blockIdx.x / ipc);
    const int64_t rr = (int64_t)blockIdx.x - (int64_t)chunk * ipc;
    const int64_t q = (rr & 7) * (ipc >> 3) + (rr >> 3);
    if (chunk >= a.nchunks || q >= a.num_items) return;  // uniform over the work-group
    const int64_t g0 = a.goff[q];
    const int64_t nslabs = a.goff[q + 1] - g0;
    const int64_t n0 = a.col_base + (int64_t)chunk * NC;

    const __amdgpu_buffer_rsrc_t rsC = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.cols + g0 * 16), (short)0, (int)(nslabs * 64), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsH = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.hdr + g0 * G * 12), (short)0, (int)(nslabs * G * 48), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsV =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.pvals), (short)0, (int)a.pv_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsX =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.x), (short)0, (int)a.x_bytes, 0x00020000);

    // gather instruction i of this wave covers its row segments 8 i .. 8 i + 7;
    // lane l takes segment 8 i + l / 8 (past the last, PAD earlier: the same
    // row, since PAD is a multiple of RPW): staged row and first element
    auto seg_of = [&](int i) { const int si = 8 * i + (lane >> 3); return si < NSEG ? si : si - PAD; };
    auto row_of = [&](int i) { return wave * RPW + seg_of(i) % RPW; };
    auto elem_of = [&](int i) { return 64 * (seg_of(i) / RPW) + 8 * (lane & 7); };
    bool lcol[NLD];
    uint32_t colb[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        lcol[i] = n0 + elem_of(i) < a.n_cols;
        colb[i] = lcol[i] ? (uint32_t)((n0 + elem_of(i)) * 2) : 0u;
    }
    const uint32_t ldxb = (uint32_t)(a.ldx * 2);
    const uint32_t xr = (uint32_t)a.x_rows;
    const int ag = lane >> 4;
    const int ar = lane & 15;
    const int tr_off = (4 * ag + ((lane & 15) >> 2)) * PITCH + 4 * (lane & 3);
    const uint32_t h_lane = (uint32_t)(ar >> 2) * 12;
    const uint32_t bitoff = (uint32_t)((ar & 3) * 16 + 4 * ag);

    // the lane's column indices of slab s: rows lane/8 and 8 + lane/8 (GW 1),
    // else its one staged row; past the group the range check returns 0
    auto load_cols = [&](int64_t s) -> ColV {
        if constexpr (GW == 1) {
            const uint32_t off = (uint32_t)(s * 64) + (uint32_t)(lane >> 3) * 4;
            return ColV{(int32_t)__builtin_amdgcn_raw_buffer_load_b32(rsC, (int)off, 0, kAPolicy),
                        (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rsC, (int)(off + 32), 0, kAPolicy)};
        } else {
            const uint32_t off = (uint32_t)(s * 64) + (uint32_t)(wave * RPW + (lane >> 3) % RPW) * 4;
            return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rsC, (int)off, 0, kAPolicy);
        }
    };
    auto load_x = [&](const ColV cv, u32x4_t* regs) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            int32_t c;
            if constexpr (GW == 1) c = cv[i & 1]; else c = cv;
            const bool ok = lcol[i] && (uint32_t)c < xr;
            const uint32_t row = ok ? (uint32_t)c : xr;  // row x_rows lies past the resource
            regs[i] = __builtin_amdgcn_raw_buffer_load_b128(rsX, (int)(__umul24(row, ldxb) + colb[i]), 0, 0);
        }
    };
    // window wi's 48-byte sub-tile header in slab s: in every quad of lanes
    // (one row group: lanes 4g..4g+3 of each row of 16) the first three
    // load the group's {mask_lo, mask_hi, start}, one word each, and
    // broadcast them over the quad (DPP quad permutes: no LDS, no SMEM)
    const uint32_t hword = (uint32_t)(3 * ((lane & 15) >> 2) + ((lane & 3) < 2 ? (lane & 3) : 2)) * 4;
    auto load_hdr = [&](int64_t s, int wi) -> uint32_t {
        return __builtin_amdgcn_raw_buffer_load_b32(rsH, (int)((uint32_t)((s * G + wave * WPW + wi) * 48) + hword), 0, kAPolicy);
    };
    auto lane_hdr = [&](const uint32_t raw) -> u32x3_t {
        return u32x3_t{(uint32_t)__builtin_amdgcn_mov_dpp((int)raw, 0x00, 0xf, 0xf, false),
                       (uint32_t)__builtin_amdgcn_mov_dpp((int)raw, 0x55, 0xf, 0xf, false),
                       (uint32_t)__builtin_amdgcn_mov_dpp((int)raw, 0xaa, 0xf, 0xf, false)};
    };
    auto load_a = [&](const u32x3_t h) -> u32x4_t {
        const uint64_t m = ((uint64_t)h[1] << 32) | h[0];
        const uint32_t below = (uint32_t)__builtin_popcountll(m & ((1ull << bitoff) - 1));
        const uint32_t nib = (uint32_t)(m >> bitoff) & 15u;
        const uint32_t hidx = h[2] + below;
        const uint32_t off = nib ? (hidx & ~1u) * 2u : 0x80000000u;  // empty: no read
        const u32x3_t d = __builtin_amdgcn_raw_buffer_load_b96(rsV, (int)off, 0, kAPolicy);
        return u32x4_t{d[0], d[1], d[2], nib | ((hidx & 1u) << 4)};
    };
    auto decode = [&](const u32x4_t v) -> short4_t {
        const uint32_t info = v[3];
        const uint32_t sh = (info >> 4) * 16u;
        const uint32_t r0 = __builtin_amdgcn_alignbit(v[1], v[0], sh);
        const uint32_t r1 = __builtin_amdgcn_alignbit(v[2], v[1], sh);
        const uint32_t b0 = info & 1u, b1 = (info >> 1) & 1u, b2 = (info >> 2) & 1u, b3 = (info >> 3) & 1u;
        const uint32_t k2 = b0 + b1, k3 = k2 + b2;
        const uint32_t s0 = b0 ? 0x0100u : 0x0c0cu;
        const uint32_t s1 = b1 ? 0x0100u + 0x0202u * b0 : 0x0c0cu;
        const uint32_t s2 = b2 ? 0x0100u + 0x0202u * k2 : 0x0c0cu;
        const uint32_t s3 = b3 ? 0x0100u + 0x0202u * k3 : 0x0c0cu;
        return __builtin_bit_cast(short4_t, u32x2_t{__builtin_amdgcn_perm(r1, r0, s0 | (s1 << 16)),
                                                    __builtin_amdgcn_perm(r1, r0, s2 | (s3 << 16))});
    };

    float4_t acc[WPW][NBLK];
#pragma unroll
    for (int w = 0; w < WPW; ++w)
#pragma unroll
        for (int b = 0; b < NBLK; ++b) acc[w][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](int buf, const u32x4_t* xb, const u32x4_t* av) {
        S* st = stage_all + buf * (16 * PITCH);
#pragma unroll
        for (int i = 0; i < NLD; ++i) *reinterpret_cast<u32x4_t*>(&st[row_of(i) * PITCH + elem_of(i)]) = xb[i];
        if constexpr (GW > 1) {
            __syncthreads();
        } else {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        short4_t af[WPW];
#pragma unroll
        for (int w = 0; w < WPW; ++w) af[w] = decode(av[w]);
#pragma unroll
        for (int b = 0; b < NBLK; ++b) {
            lds_ptr_t p = (lds_ptr_t)(st + tr_off + 16 * b);
            if constexpr (XT == GRWS_F16) {
                const half4_t bf =
                    __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4f16_t*)p));
#pragma unroll
                for (int w = 0; w < WPW; ++w)
                    acc[w][b] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, af[w]), bf,
                                                                      acc[w][b], 0, 0, 0);
            } else {
                const short4_t bf =
                    __builtin_bit_cast(short4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4bf16_t*)p));
#pragma unroll
                for (int w = 0; w < WPW; ++w)
                    acc[w][b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(af[w], bf, acc[w][b], 0, 0, 0);
            }
        }
        if constexpr (GW == 1) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    };

    if (nslabs > 0 && xr > 0) {  // uniform over the work-group
        // X rows and A values PF slabs ahead of the slab multiplied (ring of
        // R); the column indices and headers they depend on DC slabs ahead
        // (ring of RC, a multiple of R): both stream from memory once, and
        // one slab's work is too short to cover their latency (two waves
        // per group, up to 16 column blocks: c3 N = 256 2.31 against 2.39 ms).
        // With 20 blocks a slab's work covers it, and with four waves the
        // deeper ring's registers cost a wave per SIMD (both measured slower)
        constexpr int DC = (GW == 2 && NBLK < 20) ? PF + 2 : PF + 1;
        // a slot is rewritten DC slabs on: RC must exceed DC - PF so that no
        // slot of a pending slab (PF .. DC - 1 ahead) is overwritten
        constexpr int RC = (DC - PF + R) / R * R;
        static_assert(RC > DC - PF && RC >= PF && RC % R == 0, "column ring");
        u32x4_t xbuf[R][NLD];
        u32x4_t abuf[R][WPW];
        ColV cring[RC];
        uint32_t hring[RC][WPW];
        // slab k's indices live in slot k mod RC: the first PF slabs' are
        // used here, before slabs PF .. DC - 1 take their slots
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            cring[k] = load_cols(k);
#pragma unroll
            for (int w = 0; w < WPW; ++w) hring[k][w] = load_hdr(k, w);
        }
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            load_x(cring[k], xbuf[k]);
#pragma unroll
            for (int w = 0; w < WPW; ++w) abuf[k][w] = load_a(lane_hdr(hring[k][w]));
        }
#pragma unroll
        for (int k = PF; k < DC; ++k) {
            cring[k % RC] = load_cols(k);
#pragma unroll
            for (int w = 0; w < WPW; ++w) hring[k % RC][w] = load_hdr(k, w);
        }
        auto step = [&](const int u, const int64_t s) {  // u = s mod RC
            const int cd = (u + DC) % RC, cp = (u + PF) % RC, xp = (u + PF) % R;
            cring[cd] = load_cols(s + DC);
#pragma unroll
            for (int w = 0; w < WPW; ++w) hring[cd][w] = load_hdr(s + DC, w);
            load_x(cring[cp], xbuf[xp]);
#pragma unroll
            for (int w = 0; w < WPW; ++w) abuf[xp][w] = load_a(lane_hdr(hring[cp][w]));
            consume(NST > 1 ? (int)(s & 1) : 0, xbuf[u % R], abuf[u % R]);
        };
        const int64_t nturns = nslabs / RC;
        int64_t s = 0;
        for (int64_t t = 0; t < nturns; ++t) {
#pragma unroll
            for (int u = 0; u < RC; ++u) {
                step(u, s);
                ++s;
            }
        }
        const int rest = (int)(nslabs - nturns * RC);
#pragma unroll
        for (int u = 0; u < RC - 1; ++u) {
            if (u < rest) step(u, s);
            ++s;
        }
    }
#pragma unroll
    for (int w = 0; w < WPW; ++w) {
        const int64_t win = q * G + wave * WPW + w;
        if (win < a.num_windows) spmm_epilogue<XT, NBLK, 1>(a, acc[w], stage_all, 0, lane, win, -1, chunk, n0);
    }
}

// Grouped tiles of 4 windows, slabs taken in pairs: v_mfma_f32_16x16x32
// issues at the rate of v_mfma_f32_16x16x16 on gfx950 (measured: 110G
// instructions/s either way, 1.7-1.8 against 0.92 PFLOP/s f16), so one
// instruction multiplies two consecutive slabs of the same layout.  Four
// waves per group, one window each.  Per pair p the waves gather its 32 X
// rows into LDS: slab 2p into stage rows 0..15, slab 2p + 1 into 16..31,
// wave h the rows 4h..4h+3 of each slab (lane l the row of slab half
// l / 32 at position 4h + (l / 8) % 4, 8 lanes per 128-byte segment, one
// gather instruction per 64 columns); one barrier; then per 16-column
// block two transposing LDS reads (stage rows 8g..8g+3 and 8g+4..8g+7 for
// lane group g) make the B operand of one MFMA.  Lane (g, r) of the A
// operand holds row r, columns 8 (g & 1) .. + 7 of slab 2p + g / 2: two
// nibbles of that slab's row-group mask, each decoded as the 4-slot runs of
// the packed tiles.  A group with an odd slab count ends with half a pair:
// the missing slab's headers read as empty (range check) and its X rows
// as the zero row.  Double-buffered stage, one barrier per pair (a buffer
// is written again two pairs later, after every wave passed the barrier in
// between).  The sums take each row's columns in ascending order, 32 per
// MFMA step.
template <int XT, int NBLK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NBLK == 20 ? 3 : 1, 8))) void spmm_grp2_kernel(
    SpmmArgs a) {
    static_assert(XT == GRWS_F16 || XT == GRWS_BF16, "grouped tiles: 16-bit X and values");
    static_assert(NBLK == 8 || NBLK == 16 || NBLK == 20, "column blocks per chunk");
    constexpr int G = 4;
    constexpr int NC = NBLK * 16;
    constexpr int NLD = NC / 64;  // gather instructions per wave and pair
    constexpr int PITCH = NC + 16;
    using S = typename XTraits<XT>::S;
    typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
    typedef short short8_t __attribute__((ext_vector_type(8)));
    typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
    __shared__ __attribute__((aligned(16))) S stage_all[2 * 32 * PITCH];

    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    // chunk-major: every XCD walks chunk 0's groups (its own range), then chunk 1's
    const int64_t ipc = (a.num_items + 7) & ~(int64_t)7;
    const int chunk = (int)(blockIdx.x / ipc);
    const int64_t rr = (int64_t)blockIdx.x - (int64_t)chunk * ipc;
    const int64_t q = (rr & 7) * (ipc >> 3) + (rr >> 3);
    if (chunk >= a.nchunks || q >= a.num_items) return;  // uniform over the work-group
    const int64_t g0 = a.goff[q];
    const int64_t nslabs = a.goff[q + 1] - g0;
    const int64_t npairs = (nslabs + 1) >> 1;
    const int64_t n0 = a.col_base + (int64_t)chunk * NC;

    const __amdgpu_buffer_rsrc_t rsC = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.cols + g0 * 16), (short)0, (int)(nslabs * 64), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsH = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.hdr + g0 * G * 12), (short)0, (int)(nslabs * G * 48), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsV =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.pvals), (short)0, (int)a.pv_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsX =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.x), (short)0, (int)a.x_bytes, 0x00020000);

    // the lane's gathered row: slab half hx of the pair, position 4 wave + r4
    // in that slab, staged row srow; gather instruction i reads its columns
    // 64 i + 8 (lane % 8) .. + 7 of the chunk
    const int hx = lane >> 5, r4 = (lane >> 3) & 3;
    const int srow = 16 * hx + 4 * wave + r4;
    const uint32_t col_off = (uint32_t)(4 * wave + r4) * 4;
    bool lcol[NLD];
    uint32_t colb[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int64_t e = n0 + 64 * i + 8 * (lane & 7);
        lcol[i] = e < a.n_cols;
        colb[i] = lcol[i] ? (uint32_t)(e * 2) : 0u;
    }
    const uint32_t ldxb = (uint32_t)(a.ldx * 2);
    const uint32_t xr = (uint32_t)a.x_rows;
    const int ag = lane >> 4;
    const int ar = lane & 15;
    const int tr0 = (8 * ag + (ar >> 2)) * PITCH + 4 * (ar & 3);
    const int tr1 = tr0 + 4 * PITCH;
    const int ha = ag >> 1;  // the slab of the pair the lane's A operand comes from
    const uint32_t bitoff = (uint32_t)((ar & 3) * 16 + 8 * (ag & 1));
    const uint32_t hword = (uint32_t)(3 * (ar >> 2) + ((lane & 3) < 2 ? (lane & 3) : 2)) * 4;

    // column index of the lane's row in pair p; -1 (the zero row) for the
    // missing slab of a group's last pair
    auto load_col = [&](int64_t p) -> int32_t {
        const int64_t sl = 2 * p + hx;
        const int32_t c =
            (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rsC, (int)((uint32_t)(sl * 64) + col_off), 0, kAPolicy);
        return sl < nslabs ? c : -1;
    };
    auto load_x = [&](const int32_t c, u32x4_t* regs) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const bool ok = lcol[i] && (uint32_t)c < xr;
            const uint32_t row = ok ? (uint32_t)c : xr;  // row x_rows lies past the resource
            regs[i] = __builtin_amdgcn_raw_buffer_load_b128(rsX, (int)(__umul24(row, ldxb) + colb[i]), 0, 0);
        }
    };
    // the window's 48-byte sub-tile header in slab 2p + ha: the first three
    // lanes of each quad load the row group's {mask_lo, mask_hi, start}, one
    // word each, broadcast over the quad by DPP quad permutes (a quad shares
    // its row group and its slab); past the group the range check reads 0
    auto load_hdr = [&](int64_t p) -> uint32_t {
        return __builtin_amdgcn_raw_buffer_load_b32(
            rsH, (int)((uint32_t)(((2 * p + ha) * G + wave) * 48) + hword), 0, kAPolicy);
    };
    auto lane_hdr = [&](const uint32_t raw) -> u32x3_t {
        return u32x3_t{(uint32_t)__builtin_amdgcn_mov_dpp((int)raw, 0x00, 0xf, 0xf, false),
                       (uint32_t)__builtin_amdgcn_mov_dpp((int)raw, 0x55, 0xf, 0xf, false),
                       (uint32_t)__builtin_amdgcn_mov_dpp((int)raw, 0xaa, 0xf, 0xf, false)};
    };
    // the lane's 8 slots as two 4-slot runs: 12-byte reads from the even
    // value index at or below each run's first value, with the run's mask
    // nibble and the odd-start flag beside them (an empty run reads nothing)
    auto load_a = [&](const u32x3_t h, u32x4_t* out) {
        const uint64_t m = ((uint64_t)h[1] << 32) | h[0];
        const uint32_t below = (uint32_t)__builtin_popcountll(m & ((1ull << bitoff) - 1));
        const uint32_t byte = (uint32_t)(m >> bitoff) & 255u;
        const uint32_t nib0 = byte & 15u, nib1 = byte >> 4;
        const uint32_t i0 = h[2] + below;
        const uint32_t i1 = i0 + (uint32_t)__builtin_popcount(nib0);
        const uint32_t off0 = nib0 ? (i0 & ~1u) * 2u : 0x80000000u;
        const uint32_t off1 = nib1 ? (i1 & ~1u) * 2u : 0x80000000u;
        const u32x3_t d0 = __builtin_amdgcn_raw_buffer_load_b96(rsV, (int)off0, 0, kAPolicy);
        const u32x3_t d1 = __builtin_amdgcn_raw_buffer_load_b96(rsV, (int)off1, 0, kAPolicy);
        out[0] = u32x4_t{d0[0], d0[1], d0[2], nib0 | ((i0 & 1u) << 4)};
        out[1] = u32x4_t{d1[0], d1[1], d1[2], nib1 | ((i1 & 1u) << 4)};
    };
    auto decode = [&](const u32x4_t v) -> short4_t {
        const uint32_t info = v[3];
        const uint32_t sh = (info >> 4) * 16u;
        const uint32_t r0 = __builtin_amdgcn_alignbit(v[1], v[0], sh);
        const uint32_t r1 = __builtin_amdgcn_alignbit(v[2], v[1], sh);
        const uint32_t b0 = info & 1u, b1 = (info >> 1) & 1u, b2 = (info >> 2) & 1u, b3 = (info >> 3) & 1u;
        const uint32_t k2 = b0 + b1, k3 = k2 + b2;
        const uint32_t s0 = b0 ? 0x0100u : 0x0c0cu;
        const uint32_t s1 = b1 ? 0x0100u + 0x0202u * b0 : 0x0c0cu;
        const uint32_t s2 = b2 ? 0x0100u + 0x0202u * k2 : 0x0c0cu;
        const uint32_t s3 = b3 ? 0x0100u + 0x0202u * k3 : 0x0c0cu;
        return __builtin_bit_cast(short4_t, u32x2_t{__builtin_amdgcn_perm(r1, r0, s0 | (s1 << 16)),
                                                    __builtin_amdgcn_perm(r1, r0, s2 | (s3 << 16))});
    };

    float4_t acc[NBLK];
#pragma unroll
    for (int b = 0; b < NBLK; ++b) acc[b] = float4_t{0.f, 0.f, 0.f, 0.f};

    // pair p's X rows into stage buffer p & 1 (they were loaded one step
    // before); the caller issues the next pair's gathers into the same
    // registers before the barrier, so they fly during this pair's MFMAs
    auto stage_x = [&](int buf, const u32x4_t* xb) {
        S* st = stage_all + buf * (32 * PITCH);
#pragma unroll
        for (int i = 0; i < NLD; ++i)
            *reinterpret_cast<u32x4_t*>(&st[srow * PITCH + 64 * i + 8 * (lane & 7)]) = xb[i];
    };
    auto multiply = [&](int buf, const u32x4_t* av) {
        S* st = stage_all + buf * (32 * PITCH);
        const short8_t af = __builtin_shufflevector(decode(av[0]), decode(av[1]), 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int b = 0; b < NBLK; ++b) {
            lds_ptr_t p0 = (lds_ptr_t)(st + tr0 + 16 * b);
            lds_ptr_t p1 = (lds_ptr_t)(st + tr1 + 16 * b);
            if constexpr (XT == GRWS_F16) {
                const half4_t lo =
                    __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4f16_t*)p0));
                const half4_t hi =
                    __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4f16_t*)p1));
                const half8_t bf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af), bf, acc[b], 0, 0, 0);
            } else {
                const short4_t lo =
                    __builtin_bit_cast(short4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4bf16_t*)p0));
                const short4_t hi =
                    __builtin_bit_cast(short4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4bf16_t*)p1));
                const short8_t bf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af),
                                                                 __builtin_bit_cast(bf16x8_t, bf), acc[b], 0, 0, 0);
            }
        }
    };

    if (npairs > 0 && xr > 0) {  // uniform over the work-group
        // X rows and A values one pair ahead of the pair multiplied (one X
        // register set, two A sets), the column indices and headers they
        // depend on two pairs ahead (ring of 2)
        u32x4_t xbuf[NLD];
        u32x4_t abuf[2][2];
        int32_t cring[2];
        uint32_t hring[2];
        cring[0] = load_col(0);
        hring[0] = load_hdr(0);
        load_x(cring[0], xbuf);
        load_a(lane_hdr(hring[0]), abuf[0]);
        cring[1] = load_col(1);
        hring[1] = load_hdr(1);
        auto step = [&](const int u, const int64_t p) {  // u = p mod 2
            stage_x(u, xbuf);
            cring[u] = load_col(p + 2);
            hring[u] = load_hdr(p + 2);
            load_x(cring[u ^ 1], xbuf);
            load_a(lane_hdr(hring[u ^ 1]), abuf[u ^ 1]);
            __syncthreads();
            multiply(u, abuf[u]);
        };
        int64_t p = 0;
        for (; p + 1 < npairs; p += 2) {
            step(0, p);
            step(1, p + 1);
        }
        if (p < npairs) step(0, p);
    }
    const int64_t win = q * G + wave;
    if (win < a.num_windows) spmm_epilogue<XT, NBLK, 1>(a, acc, stage_all, 0, lane, win, -1, chunk, n0);
}

// The slab-pair kernel with X staged by direct loads into LDS
// (buffer_load_dwordx4 ... lds): the gathered rows go from the L2 straight
// into the stage, not through registers and LDS writes, which frees the
// 20 staging registers and 5 LDS writes per pair.  Lane l of such a load
// writes its 16 bytes at the instruction's LDS base + 16 l (a lane past the
// buffer resource writes zeros: the zero row), so the stage is blocked:
// wave h's load i fills a 1 KiB block of 8 rows (rows 4h..4h+3 of each slab
// of the pair) x 64 columns, row k of the block at 128 k, its 16-byte
// segment s at position (s + 2 (k mod 4)) mod 8: the four rows a
// transposing read takes then cover all 128 bytes of the banks once.  The
// two stage buffers are separate arrays, so the compiler can tell that a
// load into one does not feed the reads of the other.  One barrier per
// pair: each wave waits for its own loads (s_waitcnt), then the barrier
// makes every wave's rows visible and tells that the other buffer is no
// longer read; the next pair's loads go into it after the barrier.  Same
// sums, same order as spmm_grp2_kernel.  320-column chunks are held to
// three waves per SIMD (40 KiB of LDS would allow four, and the scheduler
// then serialised every MFMA behind its own LDS reads to fit 128 VGPRs);
// scheduling-group barriers keep the reads four blocks ahead of the MFMAs.
// The kernel must not spill: a build that did (scratch reloads beside the
// accumulators) summed wrongly, and a test checks the code objects for it.
template <int XT, int NBLK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NBLK == 20 ? 3 : 1, NBLK == 20 ? 3 : 8))) void spmm_grp2d_kernel(
    SpmmArgs a) {
    static_assert(XT == GRWS_F16 || XT == GRWS_BF16, "grouped tiles: 16-bit X and values");
    static_assert(NBLK == 8 || NBLK == 16 || NBLK == 20, "column blocks per chunk");
    constexpr int G = 4;
    constexpr int NC = NBLK * 16;
    constexpr int NLD = NC / 64;  // direct loads per wave and pair
    using S = typename XTraits<XT>::S;
    typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
    typedef short short8_t __attribute__((ext_vector_type(8)));
    typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) char lds_char_t;
    __shared__ __attribute__((aligned(1024))) S st0[32 * NC];
    __shared__ __attribute__((aligned(1024))) S st1[32 * NC];

    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int64_t ipc = (a.num_items + 7) & ~(int64_t)7;
    const int chunk = (int)(blockIdx.x / ipc);
    const int64_t rr = (int64_t)blockIdx.x - (int64_t)chunk * ipc;
    const int64_t q = (rr & 7) * (ipc >> 3) + (rr >> 3);
    if (chunk >= a.nchunks || q >= a.num_items) return;  // uniform over the work-group
    const int64_t g0 = a.goff[q];
    const int64_t nslabs = a.goff[q + 1] - g0;
    const int64_t npairs = (nslabs + 1) >> 1;
    const int64_t n0 = a.col_base + (int64_t)chunk * NC;

    const __amdgpu_buffer_rsrc_t rsC = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.cols + g0 * 16), (short)0, (int)(nslabs * 64), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsH = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.hdr + g0 * G * 12), (short)0, (int)(nslabs * G * 48), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsV =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.pvals), (short)0, (int)a.pv_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsX =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.x), (short)0, (int)a.x_bytes, 0x00020000);

    // the lane's gathered row: slab half hx of the pair, position 4 wave + r4
    // in that slab (block row k = 4 hx + r4 = lane / 8); block position
    // lane % 8 holds column segment (lane % 8 - 2 r4) mod 8 of each 64
    const int hx = lane >> 5, r4 = (lane >> 3) & 3;
    const uint32_t col_off = (uint32_t)(4 * wave + r4) * 4;
    const int seg = ((lane & 7) - 2 * r4) & 7;
    // load i reads columns e0 + 64 i .. + 7 (bytes 2 e0 + 128 i), if below n_cols
    const int64_t e0 = n0 + 8 * seg;
    const uint32_t colb0 = (uint32_t)(e0 * 2);
    const int32_t nvalid = (int32_t)(a.n_cols - e0 > 64 * NLD ? 64 * NLD : a.n_cols - e0);  // < 64 i: past n_cols
    const uint32_t ldxb = (uint32_t)(a.ldx * 2);
    const uint32_t xr = (uint32_t)a.x_rows;
    const int ag = lane >> 4;
    const int ar = lane & 15;
    // transposing reads: lane (ag, ar) reads row ar / 4 of block rows
    // 4 (ag / 2) .. + 3 in wave block 2 (ag % 2) (rows 8 ag .. 8 ag + 3 of
    // the 32-row stage; + NLD blocks for rows 8 ag + 4 ..), 8 bytes at
    // column 16 b + 4 (ar % 4); per b % 4 the byte offset in the block
    uint32_t troff[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int k = 4 * (ag >> 1) + (ar >> 2);
        const int s = 2 * m + ((ar & 3) >> 1);
        troff[m] = (uint32_t)((2 * (ag & 1) * NLD) * 1024 + 128 * k + 16 * ((s + 2 * (ar >> 2)) & 7) + 8 * (ar & 1));
    }
    const int ha = ag >> 1;
    const uint32_t bitoff = (uint32_t)((ar & 3) * 16 + 8 * (ag & 1));
    const uint32_t hword = (uint32_t)(3 * (ar >> 2) + ((lane & 3) < 2 ? (lane & 3) : 2)) * 4;

    auto load_col = [&](int64_t p) -> int32_t {
        const int64_t sl = 2 * p + hx;
        const int32_t c =
            (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rsC, (int)((uint32_t)(sl * 64) + col_off), 0, kAPolicy);
        return sl < nslabs ? c : -1;
    };
    // pair's X rows into stage buffer `st` (a lane past the resource writes
    // the zero row)
    auto load_x = [&](S* st, const int32_t c) {
        const uint32_t rowb = __umul24((uint32_t)c < xr ? (uint32_t)c : xr, ldxb) + colb0;
        const uint32_t zrow = __umul24(xr, ldxb);  // past the resource: the zero row
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const uint32_t off = 64 * i < nvalid ? rowb + 128u * i : zrow;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsX, (lds_ptr_t)((lds_char_t*)st + (wave * NLD + i) * 1024), 16, (int)off, 0, 0, 0);
        }
    };
    auto load_hdr = [&](int64_t p) -> uint32_t {
        return __builtin_amdgcn_raw_buffer_load_b32(
            rsH, (int)((uint32_t)(((2 * p + ha) * G + wave) * 48) + hword), 0, kAPolicy);
    };
    auto lane_hdr = [&](const uint32_t raw) -> u32x3_t {
        return u32x3_t{(uint32_t)__builtin_amdgcn_mov_dpp((int)raw, 0x00, 0xf, 0xf, false),
                       (uint32_t)__builtin_amdgcn_mov_dpp((int)raw, 0x55, 0xf, 0xf, false),
                       (uint32_t)__builtin_amdgcn_mov_dpp((int)raw, 0xaa, 0xf, 0xf, false)};
    };
    auto load_a = [&](const u32x3_t h, u32x4_t* out) {
        const uint64_t m = ((uint64_t)h[1] << 32) | h[0];
        const uint32_t below = (uint32_t)__builtin_popcountll(m & ((1ull << bitoff) - 1));
        const uint32_t byte = (uint32_t)(m >> bitoff) & 255u;
        const uint32_t nib0 = byte & 15u, nib1 = byte >> 4;
        const uint32_t i0 = h[2] + below;
        const uint32_t i1 = i0 + (uint32_t)__builtin_popcount(nib0);
        const uint32_t off0 = nib0 ? (i0 & ~1u) * 2u : 0x80000000u;
        const uint32_t off1 = nib1 ? (i1 & ~1u) * 2u : 0x80000000u;
        const u32x3_t d0 = __builtin_amdgcn_raw_buffer_load_b96(rsV, (int)off0, 0, kAPolicy);
        const u32x3_t d1 = __builtin_amdgcn_raw_buffer_load_b96(rsV, (int)off1, 0, kAPolicy);
        out[0] = u32x4_t{d0[0], d0[1], d0[2], nib0 | ((i0 & 1u) << 4)};
        out[1] = u32x4_t{d1[0], d1[1], d1[2], nib1 | ((i1 & 1u) << 4)};
    };
    auto decode = [&](const u32x4_t v) -> short4_t {
        const uint32_t info = v[3];
        const uint32_t sh = (info >> 4) * 16u;
        const uint32_t r0 = __builtin_amdgcn_alignbit(v[1], v[0], sh);
        const uint32_t r1 = __builtin_amdgcn_alignbit(v[2], v[1], sh);
        const uint32_t b0 = info & 1u, b1 = (info >> 1) & 1u, b2 = (info >> 2) & 1u, b3 = (info >> 3) & 1u;
        const uint32_t k2 = b0 + b1, k3 = k2 + b2;
        const uint32_t s0 = b0 ? 0x0100u : 0x0c0cu;
        const uint32_t s1 = b1 ? 0x0100u + 0x0202u * b0 : 0x0c0cu;
        const uint32_t s2 = b2 ? 0x0100u + 0x0202u * k2 : 0x0c0cu;
        const uint32_t s3 = b3 ? 0x0100u + 0x0202u * k3 : 0x0c0cu;
        return __builtin_bit_cast(short4_t, u32x2_t{__builtin_amdgcn_perm(r1, r0, s0 | (s1 << 16)),
                                                    __builtin_amdgcn_perm(r1, r0, s2 | (s3 << 16))});
    };

    float4_t acc[NBLK];
#pragma unroll
    for (int b = 0; b < NBLK; ++b) acc[b] = float4_t{0.f, 0.f, 0.f, 0.f};

    auto multiply = [&](S* st, const u32x4_t* av) {
        const short8_t af = __builtin_shufflevector(decode(av[0]), decode(av[1]), 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int b = 0; b < NBLK; ++b) {
            lds_ptr_t p0 = (lds_ptr_t)((lds_char_t*)st + troff[b & 3] + (b >> 2) * 1024);
            lds_ptr_t p1 = (lds_ptr_t)((lds_char_t*)st + troff[b & 3] + (b >> 2) * 1024 + NLD * 1024);
            if constexpr (XT == GRWS_F16) {
                const half4_t lo =
                    __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4f16_t*)p0));
                const half4_t hi =
                    __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4f16_t*)p1));
                const half8_t bf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af), bf, acc[b], 0, 0, 0);
            } else {
                const short4_t lo =
                    __builtin_bit_cast(short4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4bf16_t*)p0));
                const short4_t hi =
                    __builtin_bit_cast(short4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4bf16_t*)p1));
                const short8_t bf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af),
                                                                 __builtin_bit_cast(bf16x8_t, bf), acc[b], 0, 0, 0);
            }
        }
        // the scheduler's order: the reads of block b + 4 go out before the
        // MFMA of block b (0x100: LDS reads, 0x008: MFMA)
        constexpr int AHEAD = 4;
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * AHEAD, 0);
#pragma unroll
        for (int b = 0; b < NBLK - AHEAD; ++b) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, AHEAD, 0);
    };

    if (npairs > 0 && xr > 0) {  // uniform over the work-group
        // pair p + 1's X rows are loaded into the other buffer while pair p
        // is multiplied; A values one pair ahead, column indices and
        // headers two pairs ahead (ring of 2)
        u32x4_t abuf[2][2];
        int32_t cring[2];
        uint32_t hring[2];
        cring[0] = load_col(0);
        hring[0] = load_hdr(0);
        load_x(st0, cring[0]);
        load_a(lane_hdr(hring[0]), abuf[0]);
        cring[1] = load_col(1);
        hring[1] = load_hdr(1);
        // the buffers are named, not selected at run time, so that each
        // read's wait covers only the loads into its own buffer
        // (unconditional loads: past the last pair they fetch nothing and
        // write zeros into the buffer no longer read; a branch around them
        // would make the compiler wait for them before the next reads)
        auto step = [&](S* cur, S* nxt, const int u, const int64_t p) {  // u = p mod 2
            // this wave's loads into `cur` have landed before the barrier:
            // the barrier itself does not wait for loads into LDS, and the
            // compiler's own wait before a read covers only the reading
            // wave's loads, not the other waves' rows of the same buffer
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();  // pair p in `cur`; every wave is done reading `nxt`
            __builtin_amdgcn_sched_barrier(0);
            cring[u] = load_col(p + 2);
            hring[u] = load_hdr(p + 2);
            load_x(nxt, cring[u ^ 1]);
            load_a(lane_hdr(hring[u ^ 1]), abuf[u ^ 1]);
            // keep the loads ahead of the multiply (the scheduler would
            // otherwise sink them to its end, leaving them no time)
            __builtin_amdgcn_sched_barrier(0);
            multiply(cur, abuf[u]);
        };
        int64_t p = 0;
        for (; p + 1 < npairs; p += 2) {
            step(st0, st1, 0, p);
            step(st1, st0, 1, p + 1);
        }
        if (p < npairs) step(st0, st1, 0, p);
        // the loads past the last pair land before the work-group ends
        __builtin_amdgcn_s_waitcnt(0);
    }
    const int64_t win = q * G + wave;
    if (win < a.num_windows) spmm_epilogue<XT, NBLK, 1>(a, acc, st0, 0, lane, win, -1, chunk, n0);
}

// Sums the partial slots of each split window in slot order (deterministic).
// One wave per 256 floats of a (split window, chunk) block: NBLK waves per
// block, lane l owns 4 consecutive floats (one row, 4 columns).  A hub
// window split into hundreds of slots would otherwise serialise one load
// latency per slot; here the loads of 8 slots are in flight at once and are
// added in slot order afterwards (same order, same result).
template <int XT, int NBLK>
__global__ __launch_bounds__(64) void spmm_fixup_kernel(const int32_t* __restrict__ split, int64_t num_split,
                                                        const float* __restrict__ partials, int32_t nchunks,
                                                        void* y, int64_t ldy, int64_t N, int64_t col_base,
                                                        const void* res, int64_t ldr, int64_t res_rows) {
    constexpr int NC = NBLK * 16;
    constexpr int U = 8;
    const int64_t blk = blockIdx.x / NBLK;  // (split window, chunk)
    const int sub = (int)(blockIdx.x % NBLK);
    const int64_t si = blk / nchunks;
    const int chunk = (int)(blk % nchunks);
    if (si >= num_split) return;
    const int64_t w = split[3 * si];
    const int64_t first = split[3 * si + 1];
    const int cnt = split[3 * si + 2];
    const int e = 4 * (sub * 64 + (int)threadIdx.x);  // first of the lane's 4 floats in the 16 x NC block
    const int r = e / NC, c = e % NC;
    const int64_t n0 = col_base + (int64_t)chunk * NC;
    const float4_t* p = reinterpret_cast<const float4_t*>(partials + (first * nchunks + chunk) * (16 * NC) + e);
    const int64_t stride = (int64_t)nchunks * (16 * NC) / 4;  // float4s between consecutive slots
    float4_t s = float4_t{0.f, 0.f, 0.f, 0.f};
    int k = 0;
    for (; k + U <= cnt; k += U) {
        float4_t t[U];
#pragma unroll
        for (int j = 0; j < U; ++j) t[j] = __builtin_nontemporal_load(p + (k + j) * stride);
#pragma unroll
        for (int j = 0; j < U; ++j) s += t[j];
    }
    for (; k < cnt; ++k) s += __builtin_nontemporal_load(p + k * stride);
    const int64_t row = w * 16 + r;
    const int64_t o = row * ldy + n0 + c;
    const bool add = res && row < res_rows;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (n0 + c + i < N) store_out<XT>(y, o + i, add ? s[i] + load_res<XT>(res, row * ldr + n0 + c + i) : s[i]);
}

// ---------------------------------------------------------------------------
// plan construction
// ---------------------------------------------------------------------------
__global__ void plan_count_kernel(const int64_t* __restrict__ win_off, int64_t W, int64_t num_tiles, int TC,
                                  int S, int32_t* __restrict__ nitems, int32_t* __restrict__ nsplit,
                                  int32_t* __restrict__ nslot) {
    int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= W) return;
    int64_t t1 = win_off[w + 1], t0 = win_off[w];
    t1 = t1 < 0 ? 0 : (t1 > num_tiles ? num_tiles : t1);
    t0 = t0 < 0 ? 0 : (t0 > t1 ? t1 : t0);
    int64_t slabs = ((t1 - t0) * TC + 15) / 16;
    int64_t ni = slabs <= S ? 1 : (slabs + S - 1) / S;
    nitems[w] = (int32_t)ni;
    nsplit[w] = ni > 1 ? 1 : 0;
    nslot[w] = ni > 1 ? (int32_t)ni : 0;
}

__global__ void plan_fill_kernel(const int64_t* __restrict__ win_off, int64_t W, int64_t num_tiles, int TC, int S,
                                 const int64_t* __restrict__ item_off, const int64_t* __restrict__ split_off,
                                 const int64_t* __restrict__ slot_off, int32_t* __restrict__ items,
                                 int32_t* __restrict__ split) {
    int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= W) return;
    int64_t t1 = win_off[w + 1], t0 = win_off[w];
    t1 = t1 < 0 ? 0 : (t1 > num_tiles ? num_tiles : t1);
    t0 = t0 < 0 ? 0 : (t0 > t1 ? t1 : t0);
    int64_t slabs = ((t1 - t0) * TC + 15) / 16;
    int64_t ni = item_off[w + 1] - item_off[w];
    for (int64_t k = 0; k < ni; ++k) {
        int32_t* it = items + 4 * (item_off[w] + k);
        int64_t b = k * S, e = (k + 1) * S;
        it[0] = (int32_t)w;
        it[1] = (int32_t)b;
        it[2] = (int32_t)(e < slabs ? e : slabs);
        it[3] = ni > 1 ? (int32_t)(slot_off[w] + k) : -1;
    }
    if (ni > 1) {
        int32_t* sp = split + 3 * split_off[w];
        sp[0] = (int32_t)w;
        sp[1] = (int32_t)slot_off[w];
        sp[2] = (int32_t)ni;
    }
}

// Whether 256-column chunks pay: A is then streamed once per 256 columns
// instead of per 128, but a wave holds twice the accumulators and X
// registers (3 waves per SIMD instead of 4).  That wins while a 256-column
// slice of X stays in the 256 MB Infinity Cache (c3, 233k rows: 2.61 ms
// against 2.79 at N=256); when it cannot (c4, 2.45M rows of random ids) the
// gathers go to HBM and the extra resident waves hide more of their latency
// (7.31 ms against 7.72).
bool wide_chunks(int64_t x_rows, int32_t x_dtype) {
    return x_dtype != GRWS_F32 && x_rows * 256 * (int64_t)dtype_size(x_dtype) <= ((int64_t)256 << 20);
}

// MFMA column blocks (16 output columns each) per work-group: 128-column
// chunks, or 256 on the buffer-load path when N is a multiple of 256 and
// wide_chunks holds.  fp32 X stays at 128 (its loads carry half as many
// elements per lane).
int nblk_for(int64_t N, int32_t x_dtype, bool buffer_path, int64_t x_rows) {
    if (const int v = tune(kTuneNblk); v >= 0) {  // tuning override
        if (v == 1 || v == 2 || v == 4 || v == 8 || (v == 16 && x_dtype != GRWS_F32)) return v;
    }
    if (buffer_path && wide_chunks(x_rows, x_dtype) && N >= 256 && N % 256 == 0) return 16;
    return N <= 16 ? 1 : (N <= 32 ? 2 : (N <= 64 ? 4 : 8));
}

template <int XT, bool AF32, int TC, int NBLK, bool VECT, int WPB>
int launch_fwd(const SpmmArgs& a, hipStream_t stream) {
    const int64_t total = a.num_items * a.nchunks;
    const int64_t grid = ((total + 7) / 8) * 8;
    if (grid > INT32_MAX) return set_error(GRWS_E_INVALID, "spmm: too many work items (%lld)", (long long)total);
    hipLaunchKernelGGL((spmm_fwd_kernel<XT, AF32, TC, NBLK, VECT, WPB, 1>), dim3((unsigned)grid), dim3(64 * WPB),
                       0, stream, a);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

// Waves per work-group.  Two waves share an (item, chunk) when the launch has
// plenty of work-groups (irregular graphs with many windows gain from it);
// small launches keep one wave per work-group so the chip still fills.
int waves_for(const SpmmArgs& a, int nblk) {
    (void)nblk;
    if (const int v = tune(kTuneWaves); v == 1 || v == 2) return v;  // tuning override
    return a.num_items * a.nchunks >= 65536 ? 2 : 1;
}

template <int XT, bool AF32, int TC, int NBLK>
int dispatch_vec(const SpmmArgs& a, bool vect, hipStream_t stream) {
    const int wpb = waves_for(a, NBLK);
    if (vect) {
        if (wpb == 2) return launch_fwd<XT, AF32, TC, NBLK, true, 2>(a, stream);
        return launch_fwd<XT, AF32, TC, NBLK, true, 1>(a, stream);
    }
    if (wpb == 2) return launch_fwd<XT, AF32, TC, NBLK, false, 2>(a, stream);
    return launch_fwd<XT, AF32, TC, NBLK, false, 1>(a, stream);
}

template <int XT, bool AF32, int TC>
int dispatch_nblk(const SpmmArgs& a, int nblk, bool vect, hipStream_t stream) {
    switch (nblk) {
        case 1: return dispatch_vec<XT, AF32, TC, 1>(a, vect, stream);
        case 2: return dispatch_vec<XT, AF32, TC, 2>(a, vect, stream);
        case 4: return dispatch_vec<XT, AF32, TC, 4>(a, vect, stream);
        case 16:
            if constexpr (XT != GRWS_F32) return dispatch_vec<XT, AF32, TC, 16>(a, vect, stream);
            [[fallthrough]];
        default: return dispatch_vec<XT, AF32, TC, 8>(a, vect, stream);
    }
}

template <int XT, bool AF32>
int dispatch_tc(const SpmmArgs& a, int tc, int nblk, bool vect, hipStream_t stream) {
    return tc == 8 ? dispatch_nblk<XT, AF32, 8>(a, nblk, vect, stream)
                   : dispatch_nblk<XT, AF32, 16>(a, nblk, vect, stream);
}

template <int XT, bool AF32, int TC, int NBLK, int WPB, bool PK>
int launch_buf(const SpmmArgs& a, hipStream_t stream) {
    const int64_t total = a.num_items * a.nchunks;
    const int64_t grid = a.chunk_major ? ((a.num_items + 7) / 8) * 8 * a.nchunks : ((total + 7) / 8) * 8;
    if (grid > INT32_MAX) return set_error(GRWS_E_INVALID, "spmm: too many work items (%lld)", (long long)total);
    if constexpr (XT != GRWS_F32 && !AF32 && NBLK >= 4) {
        if (a.narrow || NBLK == 20) {
            hipLaunchKernelGGL((spmm_buf_kernel<XT, AF32, TC, NBLK, WPB, 1, PK, true>), dim3((unsigned)grid),
                               dim3(64 * WPB), 0, stream, a);
            GRWS_LAUNCH_CHECK();
            return GRWS_OK;
        }
    }
    if constexpr (NBLK == 20) {  // 320-column chunks exist on the narrow path only
        return set_error(GRWS_E_INVALID, "spmm: 320-column chunks need 16-bit X and values");
    } else {
        hipLaunchKernelGGL((spmm_buf_kernel<XT, AF32, TC, NBLK, WPB, 1, PK>), dim3((unsigned)grid), dim3(64 * WPB),
                           0, stream, a);
        GRWS_LAUNCH_CHECK();
        return GRWS_OK;
    }
}

template <int XT, bool AF32, int TC, bool PK>
int dispatch_buf(const SpmmArgs& a, int nblk, hipStream_t stream) {
    const bool two = waves_for(a, nblk) == 2;
    switch (nblk) {
        case 1:
            return two ? launch_buf<XT, AF32, TC, 1, 2, PK>(a, stream) : launch_buf<XT, AF32, TC, 1, 1, PK>(a, stream);
        case 2:
            return two ? launch_buf<XT, AF32, TC, 2, 2, PK>(a, stream) : launch_buf<XT, AF32, TC, 2, 1, PK>(a, stream);
        case 4:
            return two ? launch_buf<XT, AF32, TC, 4, 2, PK>(a, stream) : launch_buf<XT, AF32, TC, 4, 1, PK>(a, stream);
        case 20:
            if constexpr (XT != GRWS_F32 && !AF32)
                return two ? launch_buf<XT, AF32, TC, 20, 2, PK>(a, stream)
                           : launch_buf<XT, AF32, TC, 20, 1, PK>(a, stream);
            return set_error(GRWS_E_INVALID, "spmm: 320-column chunks need 16-bit X and values");
        case 16:
            if constexpr (XT != GRWS_F32)  // fp32 chunks stop at 128 columns
                return two ? launch_buf<XT, AF32, TC, 16, 2, PK>(a, stream)
                           : launch_buf<XT, AF32, TC, 16, 1, PK>(a, stream);
            [[fallthrough]];
        default:
            return two ? launch_buf<XT, AF32, TC, 8, 2, PK>(a, stream) : launch_buf<XT, AF32, TC, 8, 1, PK>(a, stream);
    }
}

// a.hdr set (packed tiles; the host checked 16x16 tiles of x-dtype values)
// selects the packed variant.
template <int XT, bool AF32>
int dispatch_buf_tc(const SpmmArgs& a, int tc, int nblk, hipStream_t stream) {
    if constexpr (!AF32) {
        if (a.hdr) return dispatch_buf<XT, false, 16, true>(a, nblk, stream);
    }
    return tc == 8 ? dispatch_buf<XT, AF32, 8, false>(a, nblk, stream)
                   : dispatch_buf<XT, AF32, 16, false>(a, nblk, stream);
}

// Whether the buffer-load kernel's 32-bit offsets cover this call: rows and
// row pitch below 2^24 (24-bit multiply), 2 (x_rows + 1) rows below 2^32 bytes,
// and every work item's A below 2^31 bytes (an item spans at most the
// plan's slabs_per_item slabs, or without a plan a whole window: at most
// A->max_window_slabs when the caller knows it, else the whole graph).
bool buffer_path_fits(const grws_bcsr* A, const grws_spmm_plan* plan, int64_t x_rows, int64_t ldx, int64_t nc,
                      size_t esz) {
    if (tune(kTuneKernel) == 1) return false;  // tuning override: the element-masked kernel
    const int64_t ldxb = ldx * (int64_t)esz;
    if (x_rows <= 0 || x_rows >= (1 << 24) || ldxb >= (1 << 24)) return false;
    if ((x_rows + 1) * ldxb + nc * (int64_t)esz >= ((int64_t)1 << 32)) return false;
    const int64_t sza = A->values_dtype == GRWS_F32 ? 4 : 2;
    const int64_t slabs = plan && plan->items      ? (int64_t)plan->slabs_per_item
                          : A->max_window_slabs > 0 ? (int64_t)A->max_window_slabs
                                                   : (A->num_tiles * A->tile_cols + 15) / 16 + 1;
    return (slabs + 4) * 256 * sza < ((int64_t)1 << 31);
}

template <int XT>
int launch_fixup(const grws_spmm_plan* plan, const SpmmArgs& a, int nblk, hipStream_t stream) {
    const int64_t grid = plan->num_split * a.nchunks * nblk;
    if (grid <= 0) return GRWS_OK;
    if (grid > INT32_MAX) return set_error(GRWS_E_INVALID, "spmm: too many split windows (%lld)",
                                           (long long)plan->num_split);
    switch (nblk) {
        case 1:
            hipLaunchKernelGGL((spmm_fixup_kernel<XT, 1>), dim3((unsigned)grid), dim3(64), 0, stream, plan->split,
                               plan->num_split, a.partials, a.nchunks, a.y, a.ldy, a.n_cols, a.col_base,
                               a.res, a.ldr, a.res_rows);
            break;
        case 2:
            hipLaunchKernelGGL((spmm_fixup_kernel<XT, 2>), dim3((unsigned)grid), dim3(64), 0, stream, plan->split,
                               plan->num_split, a.partials, a.nchunks, a.y, a.ldy, a.n_cols, a.col_base,
                               a.res, a.ldr, a.res_rows);
            break;
        case 4:
            hipLaunchKernelGGL((spmm_fixup_kernel<XT, 4>), dim3((unsigned)grid), dim3(64), 0, stream, plan->split,
                               plan->num_split, a.partials, a.nchunks, a.y, a.ldy, a.n_cols, a.col_base,
                               a.res, a.ldr, a.res_rows);
            break;
        case 16:
            hipLaunchKernelGGL((spmm_fixup_kernel<XT, 16>), dim3((unsigned)grid), dim3(64), 0, stream, plan->split,
                               plan->num_split, a.partials, a.nchunks, a.y, a.ldy, a.n_cols, a.col_base,
                               a.res, a.ldr, a.res_rows);
            break;
        case 20:
            hipLaunchKernelGGL((spmm_fixup_kernel<XT, 20>), dim3((unsigned)grid), dim3(64), 0, stream, plan->split,
                               plan->num_split, a.partials, a.nchunks, a.y, a.ldy, a.n_cols, a.col_base,
                               a.res, a.ldr, a.res_rows);
            break;
        default:
            hipLaunchKernelGGL((spmm_fixup_kernel<XT, 8>), dim3((unsigned)grid), dim3(64), 0, stream, plan->split,
                               plan->num_split, a.partials, a.nchunks, a.y, a.ldy, a.n_cols, a.col_base,
                               a.res, a.ldr, a.res_rows);
            break;
    }
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

// ---------------------------------------------------------------------------
// packed tiles
// ---------------------------------------------------------------------------
// One wave per 16x16 tile of 16-bit values; lane l holds slots 4l..4l+3
// (row l/4, columns 4(l%4)..+3).  nib = which of them are nonzero bit
// patterns; counts per lane are at most 4, so three ballots give every
// lane's exclusive prefix and the tile total.
struct PackLane {
    uint32_t v0, v1, nib, pre, total;
};

__device__ __forceinline__ PackLane pack_lane(const uint16_t* __restrict__ vals, int64_t t, int lane) {
    const u32x2_t v = *reinterpret_cast<const u32x2_t*>(vals + t * 256 + 4 * lane);
    PackLane p;
    p.v0 = v[0];
    p.v1 = v[1];
    p.nib = ((v[0] & 0xffffu) ? 1u : 0u) | ((v[0] >> 16) ? 2u : 0u) | ((v[1] & 0xffffu) ? 4u : 0u) |
            ((v[1] >> 16) ? 8u : 0u);
    const uint32_t cnt = (uint32_t)__builtin_popcount(p.nib);
    const uint64_t q1 = __ballot(cnt & 1u), q2 = __ballot(cnt & 2u), q4 = __ballot(cnt & 4u);
    auto below = [](uint64_t m) {
        return (uint32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    };
    p.pre = below(q1) + 2u * below(q2) + 4u * below(q4);
    p.total = (uint32_t)(__builtin_popcountll(q1) + 2 * __builtin_popcountll(q2) + 4 * __builtin_popcountll(q4));
    return p;
}

__global__ __launch_bounds__(256) void pack_count_kernel(const uint16_t* __restrict__ vals, int64_t num_tiles,
                                                         int32_t* __restrict__ counts) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= num_tiles) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const PackLane p = pack_lane(vals, t, lane);
    if (lane == 0) counts[t] = (int32_t)p.total;
}

// off: exclusive prefix of the counts (int64, num_tiles + 1 entries).
// Writes past num_values (a caller that passed a smaller count than
// grws_pack_tiles_count returned) are dropped.
__global__ __launch_bounds__(256) void pack_fill_kernel(const uint16_t* __restrict__ vals, int64_t num_tiles,
                                                        const int64_t* __restrict__ off, uint32_t* __restrict__ hdr,
                                                        uint16_t* __restrict__ pvals, int64_t num_values) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= num_tiles) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const PackLane p = pack_lane(vals, t, lane);
    const uint32_t base = (uint32_t)off[t] + p.pre;
    const uint16_t h[4] = {(uint16_t)(p.v0 & 0xffffu), (uint16_t)(p.v0 >> 16), (uint16_t)(p.v1 & 0xffffu),
                           (uint16_t)(p.v1 >> 16)};
    uint32_t k = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if ((p.nib >> j) & 1u) {
            if ((int64_t)base + k < num_values) pvals[base + k] = h[j];
            ++k;
        }
    }
    // the 16 lanes of row group q contribute 4 mask bits each, in slot order
    uint64_t m = (uint64_t)p.nib << (4 * (lane & 15));
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) m |= __shfl_xor(m, d, 64);
    if ((lane & 15) == 0) {
        uint32_t* o = hdr + t * 12 + (lane >> 4) * 3;
        o[0] = (uint32_t)m;
        o[1] = (uint32_t)(m >> 32);
        o[2] = base;
    }
}

}  // namespace
}  // namespace grws

using namespace grws;

extern "C" int grws_spmm_plan_capacity(int64_t num_windows, int64_t num_tiles, int32_t tile_cols,
                                       int32_t slabs_per_item, int64_t* max_items, int64_t* max_split) {
    clear_error();
    GRWS_CHECK_ARG(num_windows >= 0 && num_tiles >= 0, "plan_capacity: negative size");
    GRWS_CHECK_ARG(tile_cols == 8 || tile_cols == 16, "plan_capacity: tile_cols must be 8 or 16");
    GRWS_CHECK_ARG(slabs_per_item >= 1, "plan_capacity: slabs_per_item must be >= 1");
    GRWS_CHECK_ARG(max_items && max_split, "plan_capacity: null output");
    // sum_w ceil(slabs_w / S) <= W + sum_w slabs_w / S, and slabs_w <= T_w*tc/16 + 1
    int64_t slab_bound = (num_tiles * tile_cols) / 16 + num_windows;
    *max_items = num_windows + slab_bound / slabs_per_item + 1;
    int64_t ms = slab_bound / (int64_t)(slabs_per_item + 1) + 1;
    *max_split = ms < num_windows ? ms : num_windows;
    return GRWS_OK;
}

extern "C" int32_t grws_spmm_default_slabs(int64_t num_windows, int64_t num_tiles, int32_t tile_cols,
                                           int64_t n_cols) {
    int64_t nblk = nblk_for(n_cols > 0 ? n_cols : 1, GRWS_F16, true, 0);
    int64_t nchunks = (n_cols + nblk * 16 - 1) / (nblk * 16);
    if (nchunks < 1) nchunks = 1;
    int64_t slabs = (num_tiles * (tile_cols > 0 ? tile_cols : 16) + 15) / 16;
    // a fair share for one of ~4096 resident waves (256 CUs x 16).  Split
    // windows cost a partial write and a fixup read, so items stay long
    // enough that only hub windows split (measured: c2 best at 32 slabs,
    // c4 within 1% of its best at 512-1024, c3 slower once its ~320-tile
    // windows split)
    int64_t share = slabs * nchunks / 4096;
    int64_t s = 16;
    while (s * 2 <= share && s < (1 << 20)) s *= 2;
    (void)num_windows;
    return (int32_t)s;
}

extern "C" size_t grws_spmm_plan_workspace_bytes(int64_t num_windows) {
    Sizer s;
    for (int i = 0; i < 3; ++i) s.take<int32_t>((size_t)num_windows + 1);
    for (int i = 0; i < 3; ++i) s.take<int64_t>((size_t)num_windows + 2);
    s.used += scan_workspace_bytes(num_windows) + 256;
    return s.used;
}

extern "C" int grws_spmm_plan_build(const int64_t* window_offset, int64_t num_windows, int64_t num_tiles,
                                    int32_t tile_cols, int32_t slabs_per_item, int32_t* items, int64_t max_items,
                                    int32_t* split, int64_t max_split, void* workspace, size_t workspace_bytes,
                                    int64_t* counts_out, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(window_offset && items && counts_out, "plan_build: null pointer");
    GRWS_CHECK_ARG(num_windows >= 0 && num_tiles >= 0, "plan_build: negative size");
    GRWS_CHECK_ARG(tile_cols == 8 || tile_cols == 16, "plan_build: tile_cols must be 8 or 16");
    GRWS_CHECK_ARG(slabs_per_item >= 1, "plan_build: slabs_per_item must be >= 1");
    int64_t cap_items = 0, cap_split = 0;
    GRWS_TRY(grws_spmm_plan_capacity(num_windows, num_tiles, tile_cols, slabs_per_item, &cap_items, &cap_split));
    if (max_items < cap_items || max_split < cap_split || (cap_split > 0 && !split))
        return set_error(GRWS_E_CAPACITY, "plan_build: plan buffers too small (items %lld < %lld or split %lld < %lld)",
                         (long long)max_items, (long long)cap_items, (long long)max_split, (long long)cap_split);
    if (num_windows == 0) {
        counts_out[0] = counts_out[1] = counts_out[2] = 0;
        return GRWS_OK;
    }
    Carver cv(workspace, workspace_bytes);
    int32_t* nitems = cv.take<int32_t>(num_windows + 1);
    int32_t* nsplit = cv.take<int32_t>(num_windows + 1);
    int32_t* nslot = cv.take<int32_t>(num_windows + 1);
    int64_t* item_off = cv.take<int64_t>(num_windows + 2);
    int64_t* split_off = cv.take<int64_t>(num_windows + 2);
    int64_t* slot_off = cv.take<int64_t>(num_windows + 2);
    size_t scan_bytes = scan_workspace_bytes(num_windows);
    char* scan_ws = cv.take<char>(scan_bytes);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "plan_build: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    unsigned blocks = (unsigned)((num_windows + 255) / 256);
    hipLaunchKernelGGL(plan_count_kernel, dim3(blocks), dim3(256), 0, stream, window_offset, num_windows, num_tiles,
                       (int)tile_cols, (int)slabs_per_item, nitems, nsplit, nslot);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(nitems, item_off, num_windows, false, scan_ws, scan_bytes, stream));
    GRWS_TRY(scan_i32_to_i64(nsplit, split_off, num_windows, false, scan_ws, scan_bytes, stream));
    GRWS_TRY(scan_i32_to_i64(nslot, slot_off, num_windows, false, scan_ws, scan_bytes, stream));
    hipLaunchKernelGGL(plan_fill_kernel, dim3(blocks), dim3(256), 0, stream, window_offset, num_windows, num_tiles,
                       (int)tile_cols, (int)slabs_per_item, item_off, split_off, slot_off, items, split);
    GRWS_LAUNCH_CHECK();
    int64_t h[3];
    GRWS_HIP(hipMemcpyAsync(&h[0], item_off + num_windows, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&h[1], split_off + num_windows, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&h[2], slot_off + num_windows, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    counts_out[0] = h[0];
    counts_out[1] = h[1];
    counts_out[2] = h[2];
    return GRWS_OK;
}

namespace {
// Plan order: the item list is walked in eighths, one per XCD (work-group r
// takes item (r % 8) * per + r / 8, per = n rounded up to 8, over 8); within
// each eighth the items go longest first, so that the long items (a
// power-law graph's hub windows) do not start last and end the launch late.
// Key = eighth (bits 32..34) and 2^31 - 1 - slabs (low 32 bits): an
// ascending stable sort keeps equal lengths in window order.
__global__ void plan_order_keys_kernel(const int32_t* __restrict__ items, int64_t n, int64_t per,
                                       uint64_t* __restrict__ keys, uint32_t* __restrict__ idx,
                                       int32_t* __restrict__ copy) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int32_t w = items[4 * i], b = items[4 * i + 1], e = items[4 * i + 2], sl = items[4 * i + 3];
    const int64_t len = (int64_t)e - b;
    const uint32_t k = (uint32_t)(0x7fffffff - (len < 0 ? 0 : (len > 0x7fffffff ? 0x7fffffff : len)));
    keys[i] = ((uint64_t)(i / per) << 32) | k;
    idx[i] = (uint32_t)i;
    copy[4 * i] = w;
    copy[4 * i + 1] = b;
    copy[4 * i + 2] = e;
    copy[4 * i + 3] = sl;
}

__global__ void plan_order_gather_kernel(const int32_t* __restrict__ copy, const uint32_t* __restrict__ idx, int64_t n,
                                         int32_t* __restrict__ items) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const int64_t i = idx[j];
#pragma unroll
    for (int c = 0; c < 4; ++c) items[4 * j + c] = copy[4 * i + c];
}

struct PlanOrderWs {
    uint64_t *k, *k2;
    uint32_t *v, *v2;
    int32_t* copy;
    char* sort_ws;
    size_t sort_bytes;
};

void carve_plan_order(Carver& c, int64_t n, PlanOrderWs* w) {
    w->k = c.take<uint64_t>((size_t)n);
    w->k2 = c.take<uint64_t>((size_t)n);
    w->v = c.take<uint32_t>((size_t)n);
    w->v2 = c.take<uint32_t>((size_t)n);
    w->copy = c.take<int32_t>((size_t)n * 4);
    w->sort_bytes = radix_sort_workspace_bytes(n);
    w->sort_ws = c.take<char>(w->sort_bytes);
}
}  // namespace

extern "C" size_t grws_spmm_plan_order_workspace_bytes(int64_t num_items) {
    if (num_items <= 0) return 0;
    Sizer s;  // the takes of carve_plan_order
    s.take<uint64_t>((size_t)num_items);
    s.take<uint64_t>((size_t)num_items);
    s.take<uint32_t>((size_t)num_items);
    s.take<uint32_t>((size_t)num_items);
    s.take<int32_t>((size_t)num_items * 4);
    s.take<char>(radix_sort_workspace_bytes(num_items));
    return s.used + 256;
}

extern "C" int grws_spmm_plan_order(int32_t* items, int64_t num_items, void* workspace, size_t workspace_bytes,
                                    void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(num_items >= 0 && num_items < ((int64_t)1 << 31), "plan_order: bad item count %lld",
                   (long long)num_items);
    if (num_items <= 1) return GRWS_OK;
    GRWS_CHECK_ARG(items != nullptr, "plan_order: null items");
    Carver cv(workspace, workspace_bytes);
    PlanOrderWs w{};
    carve_plan_order(cv, num_items, &w);
    if (!cv.ok)
        return set_error(GRWS_E_CAPACITY, "plan_order: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const int64_t per = ((num_items + 7) / 8 * 8) / 8;
    const unsigned blocks = (unsigned)((num_items + 255) / 256);
    hipLaunchKernelGGL(plan_order_keys_kernel, dim3(blocks), dim3(256), 0, stream, items, num_items, per, w.k, w.v,
                       w.copy);
    GRWS_LAUNCH_CHECK();
    bool alt = false;
    GRWS_TRY(radix_sort_pairs(w.k, w.v, w.k2, w.v2, num_items, 35, w.sort_ws, w.sort_bytes, stream, &alt));
    hipLaunchKernelGGL(plan_order_gather_kernel, dim3(blocks), dim3(256), 0, stream, w.copy, alt ? w.v2 : w.v,
                       num_items, items);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

extern "C" size_t grws_spmm_workspace_bytes(const grws_spmm_plan* plan, int64_t n_cols) {
    if (!plan || plan->num_slots <= 0 || n_cols <= 0) return 0;
    // chunk widths divide 256 or are 320: this covers whichever runs
    const int64_t p256 = (n_cols + 255) / 256 * 256, p320 = (n_cols + 319) / 320 * 320;
    const int64_t padded = p256 > p320 ? p256 : p320;
    return (size_t)plan->num_slots * 16 * (size_t)padded * sizeof(float);
}

namespace {
// Packed values addressable by the kernel's 32-bit byte offsets (with the
// 12-byte reads past the last value inside the range check).
constexpr int64_t kPackMaxValues = ((int64_t)1 << 30) - 16;
// Elements of readable padding after the packed values (a lane's 12-byte
// read starts at most 1 element before its first value and spans 6).
constexpr int64_t kPackPad = 8;

int spmm_impl(const grws_bcsr* A, const grws_packed_tiles* P, const grws_spmm_plan* plan, const void* x,
              int32_t x_dtype, int64_t x_rows, int64_t ldx, int64_t n_cols, const void* res, int64_t ldr,
              int64_t res_rows, void* y, int32_t y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes,
              void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(A != nullptr, "spmm: null graph");
    GRWS_CHECK_ARG(A->tile_rows == 16, "spmm: tile_rows must be 16 (got %d)", A->tile_rows);
    GRWS_CHECK_ARG(A->tile_cols == 8 || A->tile_cols == 16, "spmm: tile_cols must be 8 or 16 (got %d)", A->tile_cols);
    GRWS_CHECK_ARG(A->num_windows >= 0 && A->num_tiles >= 0, "spmm: negative graph size");
    GRWS_CHECK_ARG(n_cols >= 0 && x_rows >= 0, "spmm: negative size");
    GRWS_CHECK_ARG(x_rows <= INT32_MAX, "spmm: x_rows exceeds int32 column range");
    if (x_dtype != GRWS_F32 && x_dtype != GRWS_F16 && x_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "spmm: unsupported x dtype %d", x_dtype);
    if (y_dtype != x_dtype) return set_error(GRWS_E_DTYPE, "spmm: y dtype must equal x dtype");
    if (A->values_dtype != GRWS_F32 && A->values_dtype != x_dtype)
        return set_error(GRWS_E_DTYPE, "spmm: values dtype must be F32 or the x dtype");
    if (P) {
        GRWS_CHECK_ARG(A->tile_cols == 16 && x_dtype != GRWS_F32 && A->values_dtype == x_dtype,
                       "spmm_packed: packed tiles need 16x16 tiles whose values have the x dtype");
        GRWS_CHECK_ARG(P->num_values >= 0 && P->num_values <= kPackMaxValues, "spmm_packed: bad num_values %lld",
                       (long long)P->num_values);
        GRWS_CHECK_ARG(A->num_tiles == 0 || (P->header && (P->values || P->num_values == 0)),
                       "spmm_packed: null packed arrays");
        GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(P->header) % 4 == 0, "spmm_packed: header not 4-byte aligned");
    }
    if (res) {
        GRWS_CHECK_ARG(ldr >= n_cols && res_rows >= 0, "spmm_residual: ldr < n_cols or negative r_rows");
        GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(res) % dtype_size(x_dtype) == 0,
                       "spmm_residual: residual not aligned to its element size");
    }
    if (A->num_windows == 0 || n_cols == 0) return GRWS_OK;
    GRWS_CHECK_ARG(A->window_offset && y, "spmm: null pointer");
    GRWS_CHECK_ARG(ldy >= n_cols, "spmm: ldy < n_cols");
    if (x_rows > 0) GRWS_CHECK_ARG(x != nullptr && ldx >= n_cols, "spmm: bad x (null or ldx < n_cols)");
    if (A->num_tiles > 0) GRWS_CHECK_ARG(A->col_indices && A->values, "spmm: null tile arrays");

    const size_t esz = dtype_size(x_dtype);
    const int64_t vec = (int64_t)(16 / esz);
    const bool vect = (n_cols % vec == 0) && (ldx % vec == 0) && ((reinterpret_cast<uintptr_t>(x) % 16) == 0);
    const bool use_buf = vect && buffer_path_fits(A, plan, x_rows, ldx, 256, esz);
    const int nblk = nblk_for(n_cols, x_dtype, use_buf, x_rows);
    const int64_t nc = nblk * 16;
    SpmmArgs a{};
    a.win_off = A->window_offset;
    a.cols = A->col_indices;
    a.vals = A->values;
    a.num_tiles = A->num_tiles;
    a.x = x;
    a.x_rows = x_rows;
    a.ldx = ldx;
    a.n_cols = n_cols;
    a.y = y;
    a.ldy = ldy;
    a.nchunks = (int32_t)((n_cols + nc - 1) / nc);
    a.res = res;
    a.ldr = ldr;
    a.res_rows = res ? res_rows : 0;
    if (plan) {
        GRWS_CHECK_ARG(plan->items != nullptr || plan->num_items == 0, "spmm: plan without items");
        a.items = plan->items;
        a.num_items = plan->num_items;
        if (plan->num_slots > 0) {
            size_t need = grws_spmm_workspace_bytes(plan, n_cols);
            if (!workspace || workspace_bytes < need)
                return set_error(GRWS_E_CAPACITY, "spmm: workspace too small (%zu < %zu)", workspace_bytes, need);
            GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "spmm: workspace not 16-byte aligned");
            a.partials = static_cast<float*>(workspace);
        }
    } else {
        a.items = nullptr;
        a.num_items = A->num_windows;
    }
    if (a.num_items == 0) return GRWS_OK;

    const bool af32 = A->values_dtype == GRWS_F32;
    const int tc = A->tile_cols;
    int st;
    if (use_buf) {
        a.x_bytes = (uint32_t)((x_rows - 1) * ldx * (int64_t)esz + n_cols * (int64_t)esz);
        a.chunk_major = 1;
        if (const int v = tune(kTuneOrder); v >= 0) a.chunk_major = v == 1;  // tuning override
        a.narrow = 1;  // 128-byte segments of 8 rows per gather where the kernel has them
        if (const int v = tune(kTuneNarrow); v >= 0) a.narrow = v == 1;      // tuning override
        if (P && A->num_tiles > 0) {  // the element-masked kernel below reads the dense values
            a.hdr = P->header;
            a.pvals = P->values;
            // a 12-byte read that runs past the end of the resource returns
            // zero as a whole, so the range covers the padding as well
            a.pv_bytes = (uint32_t)((P->num_values + kPackPad) * 2);
        }
        // N above 256 and not a multiple of it: 256-column chunks over the
        // whole multiples, then one narrower launch for the rest, so A is
        // streamed once per 256 columns and no chunk is mostly empty
        const bool forced = tune(kTuneNblk) >= 0;
        // 320-column chunks (narrow path) when they stream A fewer times than
        // 256-column chunks plus a narrower rest (N = 608: 2 passes, not 3)
        if (!forced && !af32 && x_dtype != GRWS_F32 && n_cols > 256 && n_cols % 256 != 0 &&
            x_rows * 320 * (int64_t)esz <= ((int64_t)256 << 20) && (n_cols + 319) / 320 < (n_cols + 255) / 256 &&
            (x_rows + 1) * ldx * (int64_t)esz + 320 * (int64_t)esz < ((int64_t)1 << 32) &&
            tune(kTuneC320) != 0) {
            a.col_base = 0;
            a.nchunks = (int32_t)((n_cols + 319) / 320);
            st = x_dtype == GRWS_F16 ? dispatch_buf_tc<GRWS_F16, false>(a, tc, 20, stream)
                                     : dispatch_buf_tc<GRWS_BF16, false>(a, tc, 20, stream);
            if (st == GRWS_OK && plan && plan->num_split > 0)
                st = x_dtype == GRWS_F16 ? launch_fixup<GRWS_F16>(plan, a, 20, stream)
                                         : launch_fixup<GRWS_BF16>(plan, a, 20, stream);
            return st;
        }
        const int64_t head =
            (!forced && wide_chunks(x_rows, x_dtype) && n_cols > 256 && n_cols % 256 != 0) ? n_cols / 256 * 256 : 0;
        const int64_t parts[2][2] = {{0, head > 0 ? head : n_cols}, {head, n_cols}};
        for (int pi = 0; pi < (head > 0 ? 2 : 1); ++pi) {
            const int64_t c0 = parts[pi][0], c1 = parts[pi][1];
            const int pnblk = head > 0 ? (pi == 0 ? 16 : nblk_for(c1 - c0, x_dtype, false, x_rows)) : nblk;
            const int64_t pnc = pnblk * 16;
            a.col_base = c0;
            a.nchunks = (int32_t)((c1 - c0 + pnc - 1) / pnc);
            if (x_dtype == GRWS_F32)  // fp32 X: fp32 values (checked above)
                st = dispatch_buf_tc<GRWS_F32, true>(a, tc, pnblk, stream);
            else if (x_dtype == GRWS_F16)
                st = af32 ? dispatch_buf_tc<GRWS_F16, true>(a, tc, pnblk, stream)
                          : dispatch_buf_tc<GRWS_F16, false>(a, tc, pnblk, stream);
            else
                st = af32 ? dispatch_buf_tc<GRWS_BF16, true>(a, tc, pnblk, stream)
                          : dispatch_buf_tc<GRWS_BF16, false>(a, tc, pnblk, stream);
            if (st != GRWS_OK) return st;
            if (plan && plan->num_split > 0) {
                st = x_dtype == GRWS_F32   ? launch_fixup<GRWS_F32>(plan, a, pnblk, stream)
                     : x_dtype == GRWS_F16 ? launch_fixup<GRWS_F16>(plan, a, pnblk, stream)
                                           : launch_fixup<GRWS_BF16>(plan, a, pnblk, stream);
                if (st != GRWS_OK) return st;
            }
        }
        return GRWS_OK;
    } else switch (x_dtype) {
        case GRWS_F32: st = dispatch_tc<GRWS_F32, true>(a, tc, nblk, vect, stream); break;
        case GRWS_F16:
            st = af32 ? dispatch_tc<GRWS_F16, true>(a, tc, nblk, vect, stream)
                      : dispatch_tc<GRWS_F16, false>(a, tc, nblk, vect, stream);
            break;
        default:
            st = af32 ? dispatch_tc<GRWS_BF16, true>(a, tc, nblk, vect, stream)
                      : dispatch_tc<GRWS_BF16, false>(a, tc, nblk, vect, stream);
            break;
    }
    if (st != GRWS_OK) return st;
    if (plan && plan->num_split > 0) {
        switch (x_dtype) {
            case GRWS_F32: return launch_fixup<GRWS_F32>(plan, a, nblk, stream);
            case GRWS_F16: return launch_fixup<GRWS_F16>(plan, a, nblk, stream);
            default: return launch_fixup<GRWS_BF16>(plan, a, nblk, stream);
        }
    }
    return GRWS_OK;
}
}  // namespace

namespace {
template <int XT, int NBLK, int WPW, int GW>
int launch_grp(const SpmmArgs& a, hipStream_t stream) {
    const int64_t ipc = (a.num_items + 7) & ~(int64_t)7;
    const int64_t grid = ipc * a.nchunks;
    if (grid <= 0) return GRWS_OK;
    if (grid > INT32_MAX) return set_error(GRWS_E_INVALID, "spmm_grouped: grid too large");
    // two waves per group: X rows two slabs ahead (more bytes in flight per
    // CU; measured 5.54 against 5.73 ms on c3 at N = 608)
    constexpr int PF = GW == 2 ? 2 : 1;
    hipLaunchKernelGGL((spmm_grp_kernel<XT, NBLK, WPW, GW, PF>), dim3((unsigned)grid), dim3(64 * GW), 0, stream, a);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

// Kernel shapes per group size: (windows per wave, waves per group) and the
// column blocks per chunk.  With four waves and NBLK 20 each wave's 20 row
// segments take three gather instructions (the last repeats four); WPW 4
// keeps to NBLK 8 (128 accumulator registers).
template <int XT, int NBLK>
int launch_grp2(const SpmmArgs& a, hipStream_t stream) {
    const int64_t ipc = (a.num_items + 7) & ~(int64_t)7;
    const int64_t grid = ipc * a.nchunks;
    if (grid <= 0) return GRWS_OK;
    if (grid > INT32_MAX) return set_error(GRWS_E_INVALID, "spmm_grouped: grid too large");
    if (tune(kTuneGrpDma) != 0)
        hipLaunchKernelGGL((spmm_grp2d_kernel<XT, NBLK>), dim3((unsigned)grid), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((spmm_grp2_kernel<XT, NBLK>), dim3((unsigned)grid), dim3(256), 0, stream, a);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

template <int XT>
int dispatch_grp(const SpmmArgs& a, int G, int wpw, int nblk, hipStream_t stream) {
    const int gw = G / wpw;
    // 4 windows, one per wave: slab pairs on the 16x16x32 MFMA
    if (G == 4 && wpw == 1 && tune(kTuneGrpK32) != 0) {
        if (nblk == 20) return launch_grp2<XT, 20>(a, stream);
        if (nblk == 16) return launch_grp2<XT, 16>(a, stream);
        if (nblk == 8) return launch_grp2<XT, 8>(a, stream);
    }
#define GRWS_GRP(W_, GW_, NB_) \
    if (wpw == W_ && gw == GW_ && nblk == NB_) return launch_grp<XT, NB_, W_, GW_>(a, stream)
    GRWS_GRP(1, 2, 8); GRWS_GRP(1, 2, 16); GRWS_GRP(1, 2, 20);
    GRWS_GRP(2, 1, 8); GRWS_GRP(2, 1, 16); GRWS_GRP(2, 1, 20);
    GRWS_GRP(1, 4, 8); GRWS_GRP(1, 4, 16); GRWS_GRP(1, 4, 20);
    GRWS_GRP(2, 2, 8); GRWS_GRP(2, 2, 16); GRWS_GRP(2, 2, 20);
    GRWS_GRP(4, 1, 8);
    GRWS_GRP(2, 4, 8); GRWS_GRP(2, 4, 16);
    GRWS_GRP(4, 2, 8);
#undef GRWS_GRP
    return set_error(GRWS_E_INVALID, "spmm_grouped: no kernel for group %d, %d windows per wave, %d blocks", G, wpw,
                     nblk);
}
}  // namespace

extern "C" int grws_spmm_grouped(const grws_bcsr* A, const grws_grouped_tiles* Gt, const void* x, int32_t x_dtype,
                                 int64_t x_rows, int64_t ldx, int64_t n_cols, const void* r, int64_t ldr,
                                 int64_t r_rows, void* y, int32_t y_dtype, int64_t ldy, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(A != nullptr && Gt != nullptr, "spmm_grouped: null graph or grouped tiles");
    GRWS_CHECK_ARG(A->tile_rows == 16, "spmm_grouped: tile_rows must be 16");
    if (x_dtype != GRWS_F16 && x_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "spmm_grouped: x must be F16 or BF16 (got %d)", x_dtype);
    if (y_dtype != x_dtype || A->values_dtype != x_dtype)
        return set_error(GRWS_E_DTYPE, "spmm_grouped: y and the values must have the x dtype");
    const int G = Gt->group_size;
    GRWS_CHECK_ARG(G == 2 || G == 4 || G == 8, "spmm_grouped: group_size must be 2, 4 or 8 (got %d)", G);
    GRWS_CHECK_ARG(Gt->num_groups == (A->num_windows + G - 1) / G, "spmm_grouped: %lld groups for %lld windows",
                   (long long)Gt->num_groups, (long long)A->num_windows);
    GRWS_CHECK_ARG(n_cols >= 0 && x_rows >= 0 && Gt->num_slabs >= 0 && Gt->num_values >= 0,
                   "spmm_grouped: negative size");
    GRWS_CHECK_ARG(x_rows <= Gt->num_cols, "spmm_grouped: x has %lld rows, the tiles were grouped for %lld columns",
                   (long long)x_rows, (long long)Gt->num_cols);
    GRWS_CHECK_ARG(Gt->num_values <= kPackMaxValues, "spmm_grouped: too many values (%lld)",
                   (long long)Gt->num_values);
    GRWS_CHECK_ARG(Gt->max_group_slabs >= 0 && Gt->max_group_slabs * G * 48 < ((int64_t)1 << 31),
                   "spmm_grouped: a group's headers exceed 2^31 bytes");
    if (A->num_windows == 0 || n_cols == 0) return GRWS_OK;
    GRWS_CHECK_ARG(Gt->group_offset && y, "spmm_grouped: null pointer");
    if (Gt->num_slabs > 0) GRWS_CHECK_ARG(Gt->col_indices && Gt->header, "spmm_grouped: null tile arrays");
    if (Gt->num_values > 0) GRWS_CHECK_ARG(Gt->values != nullptr, "spmm_grouped: null values");
    GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(Gt->header) % 4 == 0, "spmm_grouped: header not 4-byte aligned");
    GRWS_CHECK_ARG(ldy >= n_cols, "spmm_grouped: ldy < n_cols");
    GRWS_CHECK_ARG(x_rows > 0 && x != nullptr && ldx >= n_cols, "spmm_grouped: bad x (empty, null or ldx < n_cols)");
    GRWS_CHECK_ARG(n_cols % 8 == 0 && ldx % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0,
                   "spmm_grouped: x needs 16-byte rows (n_cols and ldx multiples of 8, 16-byte aligned)");
    GRWS_CHECK_ARG(x_rows < (1 << 24) && ldx * 2 < (1 << 24), "spmm_grouped: x exceeds 2^24 rows or row bytes");
    GRWS_CHECK_ARG((x_rows + 1) * ldx * 2 + 320 * 2 < ((int64_t)1 << 32), "spmm_grouped: x exceeds 32-bit offsets");

    if (r) {
        GRWS_CHECK_ARG(ldr >= n_cols && r_rows >= 0, "spmm_grouped: ldr < n_cols or negative r_rows");
        GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(r) % 2 == 0, "spmm_grouped: residual not 2-byte aligned");
    }

    SpmmArgs a{};
    a.res = r;
    a.ldr = ldr;
    a.res_rows = r ? r_rows : 0;
    a.cols = Gt->col_indices;
    a.hdr = Gt->header;
    a.pvals = Gt->values;
    a.pv_bytes = (uint32_t)((Gt->num_values + kPackPad) * 2);
    a.goff = Gt->group_offset;
    a.num_items = Gt->num_groups;
    a.num_windows = A->num_windows;
    a.x = x;
    a.x_rows = x_rows;
    a.ldx = ldx;
    a.n_cols = n_cols;
    a.y = y;
    a.ldy = ldy;
    a.x_bytes = (uint32_t)((x_rows - 1) * ldx * 2 + n_cols * 2);
    a.chunk_major = 1;
    // shape: windows per wave and column blocks; N above 256 not a multiple
    // of 256 runs 320-column chunks when they stream the tiles fewer times,
    // else 256-column chunks plus one narrower launch for the rest
    int wpw = G == 8 ? 2 : 1;
    int head_nblk = n_cols > 128 ? 16 : 8, tail_nblk = 8;
    if (const int v = tune(kTuneGrpWpw); v >= 0) wpw = v;  // tuning overrides
    if (const int v = tune(kTuneGrpNblk); v >= 0) head_nblk = v;
    if (wpw == 4) head_nblk = 8;
    if (wpw == 4 || G / wpw == 4) tail_nblk = 8;
    const int64_t hnc = head_nblk * 16;
    const bool c320 = head_nblk == 16 && n_cols > 256 && n_cols % 256 != 0 && (n_cols + 319) / 320 < (n_cols + 255) / 256 &&
                      (G / wpw <= 2 || (wpw == 1 && G == 4)) && tune(kTuneGrpC320) != 0;
    int st;
    if (c320) {
        a.col_base = 0;
        a.nchunks = (int32_t)((n_cols + 319) / 320);
        st = x_dtype == GRWS_F16 ? dispatch_grp<GRWS_F16>(a, G, wpw, 20, stream)
                                 : dispatch_grp<GRWS_BF16>(a, G, wpw, 20, stream);
        return st;
    }
    const int64_t head = n_cols > hnc && n_cols % hnc != 0 ? n_cols / hnc * hnc : n_cols;
    const int64_t parts[2][2] = {{0, head}, {head, n_cols}};
    for (int pi = 0; pi < (head < n_cols ? 2 : 1); ++pi) {
        const int64_t c0 = parts[pi][0], c1 = parts[pi][1];
        int nb = pi == 0 ? head_nblk : tail_nblk;
        if (pi == 1 && c1 - c0 > tail_nblk * 16) nb = head_nblk;
        a.col_base = c0;
        a.nchunks = (int32_t)((c1 - c0 + nb * 16 - 1) / (nb * 16));
        st = x_dtype == GRWS_F16 ? dispatch_grp<GRWS_F16>(a, G, wpw, nb, stream)
                                 : dispatch_grp<GRWS_BF16>(a, G, wpw, nb, stream);
        if (st != GRWS_OK) return st;
    }
    return GRWS_OK;
}

extern "C" int grws_spmm(const grws_bcsr* A, const grws_spmm_plan* plan, const void* x, int32_t x_dtype,
                         int64_t x_rows, int64_t ldx, int64_t n_cols, void* y, int32_t y_dtype, int64_t ldy,
                         void* workspace, size_t workspace_bytes, void* stream) {
    return spmm_impl(A, nullptr, plan, x, x_dtype, x_rows, ldx, n_cols, nullptr, 0, 0, y, y_dtype, ldy, workspace,
                     workspace_bytes, stream);
}

extern "C" int grws_spmm_packed(const grws_bcsr* A, const grws_packed_tiles* P, const grws_spmm_plan* plan,
                                const void* x, int32_t x_dtype, int64_t x_rows, int64_t ldx, int64_t n_cols, void* y,
                                int32_t y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
    return spmm_impl(A, P, plan, x, x_dtype, x_rows, ldx, n_cols, nullptr, 0, 0, y, y_dtype, ldy, workspace,
                     workspace_bytes, stream);
}

extern "C" int grws_spmm_residual(const grws_bcsr* A, const grws_packed_tiles* P, const grws_spmm_plan* plan,
                                  const void* x, int32_t x_dtype, int64_t x_rows, int64_t ldx, int64_t n_cols,
                                  const void* r, int64_t ldr, int64_t r_rows, void* y, int32_t y_dtype, int64_t ldy,
                                  void* workspace, size_t workspace_bytes, void* stream) {
    return spmm_impl(A, P, plan, x, x_dtype, x_rows, ldx, n_cols, r, ldr, r_rows, y, y_dtype, ldy, workspace,
                     workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// allocation-free SpMM: the split-window partials live in a library-owned
// device array instead of a caller workspace
// ---------------------------------------------------------------------------
namespace {
// Every GPU the library runs on holds one copy of this array until the
// process ends.  Host code never passes its name to a kernel (on the host it
// is only a stand-in for the symbol): the device address of each GPU's copy
// is looked up once per device and kept in scratch_ptr.
static __device__ __align__(256) unsigned char scratch[GRWS_SPMM_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch (looked up on the first
// call on that device, with it current).
int scratch_for_current_device(void** out) {
    int dev = -1;
    GRWS_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return set_error(GRWS_E_INVALID, "spmm_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        GRWS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return set_error(GRWS_E_HIP, "spmm_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GRWS_OK;
}
}  // namespace

extern "C" int grws_spmm_set_tuning(const char* name, int32_t value) {
    clear_error();
    GRWS_CHECK_ARG(name != nullptr, "spmm_set_tuning: null name");
    for (int i = 0; i < kTuneCount; ++i)
        if (strcmp(name, kTuneNames[i]) == 0) {
            g_tune[i].store(value < 0 ? -1 : value, std::memory_order_relaxed);
            return GRWS_OK;
        }
    return set_error(GRWS_E_INVALID, "spmm_set_tuning: unknown override '%s'", name);
}

extern "C" int32_t grws_spmm_get_tuning(const char* name) {
    if (!name) return -1;
    for (int i = 0; i < kTuneCount; ++i)
        if (strcmp(name, kTuneNames[i]) == 0) return g_tune[i].load(std::memory_order_relaxed);
    return -1;
}

extern "C" int grws_spmm_noalloc(const grws_bcsr* A, const grws_packed_tiles* P, const grws_spmm_plan* plan,
                                 const void* x, int32_t x_dtype, int64_t x_rows, int64_t ldx, int64_t n_cols,
                                 const void* r, int64_t ldr, int64_t r_rows, void* y, int32_t y_dtype, int64_t ldy,
                                 void* stream) {
    clear_error();
    const size_t need = grws_spmm_workspace_bytes(plan, n_cols);
    if (need > (size_t)GRWS_SPMM_NOALLOC_SCRATCH_BYTES)
        return set_error(GRWS_E_CAPACITY,
                         "spmm_noalloc: the split windows need %zu bytes of partials, above the %zu-byte scratch "
                         "(use grws_spmm_residual with a workspace, or a plan with more slabs per item)",
                         need, (size_t)GRWS_SPMM_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (need > 0) {
        // the scratch array read below is the current device's: a stream of
        // another device would reach it across devices
        int dev = 0;
        GRWS_HIP(hipGetDevice(&dev));
        hipDevice_t sdev = -1;
        const hipError_t e = hipStreamGetDevice(as_stream(stream), &sdev);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return set_error(GRWS_E_INVALID, "spmm_noalloc: cannot tell the stream's device (%s)",
                             hipGetErrorString(e));
        }
        if (sdev != dev)
            return set_error(GRWS_E_INVALID,
                             "spmm_noalloc: the stream belongs to device %d, not the current device %d "
                             "(make the stream's device current first)", (int)sdev, dev);
        GRWS_TRY(scratch_for_current_device(&ws));
    }
    // every partial a launch reads was written by the same launch's items
    // first, so the scratch needs no clearing between calls
    return spmm_impl(A, P, plan, x, x_dtype, x_rows, ldx, n_cols, r, ldr, r_rows, y, y_dtype,
                     ldy, ws, need, stream);
}

namespace {
int check_pack_graph(const grws_bcsr* A) {
    GRWS_CHECK_ARG(A != nullptr, "pack_tiles: null graph");
    GRWS_CHECK_ARG(A->tile_rows == 16 && A->tile_cols == 16, "pack_tiles: tiles must be 16x16 (got %dx%d)",
                   A->tile_rows, A->tile_cols);
    if (A->values_dtype != GRWS_F16 && A->values_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "pack_tiles: values must be F16 or BF16");
    GRWS_CHECK_ARG(A->num_tiles >= 0, "pack_tiles: negative tile count");
    if (A->num_tiles > 0) {
        GRWS_CHECK_ARG(A->values != nullptr, "pack_tiles: null values");
        GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(A->values) % 8 == 0, "pack_tiles: values not 8-byte aligned");
    }
    return GRWS_OK;
}

struct PackWs {
    int32_t* counts;
    int64_t* off;
    char* scan;
    size_t scan_bytes;
    bool ok;
    size_t used;
};

PackWs carve_pack(void* ws, size_t wsb, int64_t num_tiles) {
    Carver cv(ws, wsb);
    PackWs w;
    w.counts = cv.take<int32_t>(num_tiles + 1);
    w.off = cv.take<int64_t>(num_tiles + 2);
    w.scan_bytes = scan_workspace_bytes(num_tiles);
    w.scan = cv.take<char>(w.scan_bytes);
    w.ok = cv.ok;
    w.used = cv.used;
    return w;
}
}  // namespace

extern "C" size_t grws_pack_tiles_workspace_bytes(int64_t num_tiles) {
    if (num_tiles < 0) return 0;
    Sizer s;
    s.take<int32_t>((size_t)num_tiles + 1);
    s.take<int64_t>((size_t)num_tiles + 2);
    s.used += scan_workspace_bytes(num_tiles) + 256;
    return s.used;
}

extern "C" int grws_pack_tiles_count(const grws_bcsr* A, void* workspace, size_t workspace_bytes,
                                     int64_t* num_values, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_pack_graph(A));
    GRWS_CHECK_ARG(num_values != nullptr, "pack_tiles_count: null output");
    *num_values = 0;
    if (A->num_tiles == 0) return GRWS_OK;
    PackWs w = carve_pack(workspace, workspace_bytes, A->num_tiles);
    if (!w.ok)
        return set_error(GRWS_E_CAPACITY, "pack_tiles_count: workspace too small (%zu < %zu)", workspace_bytes, w.used);
    const int64_t blocks = (A->num_tiles + 3) / 4;
    if (blocks > INT32_MAX) return set_error(GRWS_E_INVALID, "pack_tiles_count: too many tiles");
    hipLaunchKernelGGL(pack_count_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(A->values), A->num_tiles, w.counts);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(w.counts, w.off, A->num_tiles, false, w.scan, w.scan_bytes, stream));
    int64_t total = 0;
    GRWS_HIP(hipMemcpyAsync(&total, w.off + A->num_tiles, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    *num_values = total;
    if (total > kPackMaxValues)
        return set_error(GRWS_E_CAPACITY, "pack_tiles_count: %lld nonzero values exceed the packed limit %lld",
                         (long long)total, (long long)kPackMaxValues);
    return GRWS_OK;
}

extern "C" int grws_pack_tiles_fill(const grws_bcsr* A, uint32_t* header, void* values, int64_t num_values,
                                    void* workspace, size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_pack_graph(A));
    GRWS_CHECK_ARG(num_values >= 0 && num_values <= kPackMaxValues, "pack_tiles_fill: bad num_values %lld",
                   (long long)num_values);
    if (A->num_tiles == 0) return GRWS_OK;
    GRWS_CHECK_ARG(header != nullptr && (values != nullptr || num_values == 0), "pack_tiles_fill: null output");
    GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(header) % 4 == 0, "pack_tiles_fill: header not 4-byte aligned");
    PackWs w = carve_pack(workspace, workspace_bytes, A->num_tiles);
    if (!w.ok)
        return set_error(GRWS_E_CAPACITY, "pack_tiles_fill: workspace too small (%zu < %zu)", workspace_bytes, w.used);
    const int64_t blocks = (A->num_tiles + 3) / 4;
    hipLaunchKernelGGL(pack_fill_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(A->values), A->num_tiles, w.off, header,
                       static_cast<uint16_t*>(values), num_values);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

