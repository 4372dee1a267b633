// Fused per-row epilogues of the GCN model (gfx950).
//
// 1. Activation -> LayerNorm -> dropout, the per-hidden-layer tail of the
//    reference model (models/model.py:259-264: act, self.norms[l], dropout),
//    forward and backward.  The unfused torch path makes ~6 passes over the
//    [rows x dim] activations forward (cast, ReLU, LayerNorm, dropout, cast)
//    and ~8 backward; here each direction is one pass: one wave64 per row,
//    4 consecutive elements per lane per 256 columns, statistics in fp32.
//    The dropout mask is a pure function of (seed, row, column) -- Philox4x32-10
//    (Salmon et al., SC'11), counter (row_lo, row_hi, column/4, 0), one
//    4-word block per 4 columns, element kept when its word >= p * 2^32 --
//    so the backward recomputes it instead of storing it.  dgamma / dbeta are
//    summed per work-group in registers and LDS, then over work-groups in a
//    fixed order (deterministic).
// 2. Cross-entropy over a row subset (helper/engine.py:22-41 on
//    logits[train_idx]): log-sum-exp, the label's term, mean over the rows
//    whose label is not ignore_index, and the argmax hit count, in one pass
//    over the selected rows; the backward writes softmax - onehot scaled by
//    the incoming gradient straight into the selected rows of a
//    [rows x classes] gradient.
#include "grws_internal.h"

namespace grws {
namespace {

constexpr int kBlk = 256;
constexpr int kRowsPerBlock = kBlk / kWave;

typedef float float4_t __attribute__((ext_vector_type(4)));

struct Philox4 {
    uint32_t w[4];
};

__device__ __forceinline__ Philox4 philox4(uint64_t seed, uint64_t row, uint32_t block) {
    uint32_t c0 = (uint32_t)row, c1 = (uint32_t)(row >> 32), c2 = block, c3 = 0u;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        // one 32x32->64 multiply each (v_mad_u64_u32) instead of separate
        // high and low multiplies
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
    return Philox4{{c0, c1, c2, c3}};
}

// Four consecutive elements as loaded (converted later, so a load can be
// issued an iteration ahead of its use).
template <typename T>
struct Raw4 {
    using V = uint2;
};
template <>
struct Raw4<float> {
    using V = float4_t;
};

template <typename T>
__device__ __forceinline__ typename Raw4<T>::V load_raw4(const T* p) {
    return *reinterpret_cast<const typename Raw4<T>::V*>(p);
}

template <typename T>
__device__ __forceinline__ void cvt4(const typename Raw4<T>::V& x, float* v) {
    if constexpr (std::is_same<T, float>::value) {
        v[0] = x[0], v[1] = x[1], v[2] = x[2], v[3] = x[3];
    } else {
        const T* h = reinterpret_cast<const T*>(&x);
        v[0] = to_float(h[0]), v[1] = to_float(h[1]), v[2] = to_float(h[2]), v[3] = to_float(h[3]);
    }
}

template <typename T>
__device__ __forceinline__ void load4(const T* p, float* v) {
    if constexpr (std::is_same<T, float>::value) {
        const float4_t x = *reinterpret_cast<const float4_t*>(p);
        v[0] = x[0], v[1] = x[1], v[2] = x[2], v[3] = x[3];
    } else {
        const uint2 x = *reinterpret_cast<const uint2*>(p);
        const T* h = reinterpret_cast<const T*>(&x);
        v[0] = to_float(h[0]), v[1] = to_float(h[1]), v[2] = to_float(h[2]), v[3] = to_float(h[3]);
    }
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const float* v) {
    if constexpr (std::is_same<T, float>::value) {
        *reinterpret_cast<float4_t*>(p) = float4_t{v[0], v[1], v[2], v[3]};
    } else {
        T h[4] = {from_float<T>(v[0]), from_float<T>(v[1]), from_float<T>(v[2]), from_float<T>(v[3])};
        *reinterpret_cast<uint2*>(p) = *reinterpret_cast<const uint2*>(h);
    }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 64 lanes, the same value in every lane, in a fixed order:
// within each row of 16 lanes by DPP (xor 1, xor 2 quad permutes, then
// rotations by 4 and 8), then the 4 row sums in row order.  No LDS traffic.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x124>(v);  // row_ror:4
    v += dpp_f<0x128>(v);  // row_ror:8
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return ((r0 + r1) + r2) + r3;
}

__device__ __forceinline__ uint32_t keep_threshold(float p) {
    const double t = (double)p * 4294967296.0;
    return t >= 4294967295.0 ? 0xFFFFFFFFu : (uint32_t)t;
}

// out = dropout(LayerNorm(act(z))).  One wave per row, ROWS rows in flight
// per wave (their loads are issued together, an iteration ahead), STEPS =
// ceil(dim / 256).
template <typename ZT, typename OT, int STEPS, int ROWS>
__global__ __launch_bounds__(kBlk) void act_norm_dropout_fwd_kernel(
    const ZT* __restrict__ z, int64_t ldz, int64_t rows, int dim, int act, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, float p, uint64_t seed, const uint64_t* __restrict__ seed_dev,
    OT* __restrict__ out, int64_t ldo, float* __restrict__ mean_out, float* __restrict__ rstd_out) {
    if (seed_dev) seed = *seed_dev;  // a seed drawn on the device (graph-captured callers)
    const int lane = threadIdx.x & 63;
    // wave-uniform row index: per-row scalars then go through scalar loads
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t thr = keep_threshold(p);
    const float scale = p > 0.f ? 1.0f / (1.0f - p) : 1.0f;
    const float inv_dim = 1.0f / (float)dim;
    // this lane's gamma / beta, loaded once for all its rows
    float gm[STEPS][4], bt[STEPS][4];
#pragma unroll
    for (int k = 0; k < STEPS; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = 256 * k + 4 * lane + j;
            gm[k][j] = c < dim ? gamma[c] : 0.f;
            bt[k][j] = c < dim ? beta[c] : 0.f;
        }
    const int64_t stride = (int64_t)gridDim.x * kRowsPerBlock * ROWS;
    // the next iteration's rows are loaded while this one is computed
    typename Raw4<ZT>::V raw[ROWS][STEPS];
    auto fetch = [&](int64_t rb) {
#pragma unroll
        for (int i = 0; i < ROWS; ++i)
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                const int c = 256 * k + 4 * lane;
                if (rb + i < rows && c < dim) raw[i][k] = load_raw4(z + (rb + i) * ldz + c);
                else raw[i][k] = typename Raw4<ZT>::V{};
            }
    };
    int64_t r0 = ((int64_t)blockIdx.x * kRowsPerBlock + wave) * ROWS;
    if (r0 < rows) fetch(r0);
    for (; r0 < rows; r0 += stride) {
        float x[ROWS][STEPS][4];
#pragma unroll
        for (int i = 0; i < ROWS; ++i)
#pragma unroll
            for (int k = 0; k < STEPS; ++k) cvt4<ZT>(raw[i][k], x[i][k]);
        if (r0 + stride < rows) fetch(r0 + stride);
        float mean[ROWS], rstd[ROWS];
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            float sum = 0.f;
#pragma unroll
            for (int k = 0; k < STEPS; ++k)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (act == 1) x[i][k][j] = x[i][k][j] < 0.f ? 0.f : x[i][k][j];  // NaN passes, as torch.relu
                    sum += x[i][k][j];
                }
            mean[i] = wave_sum(sum) * inv_dim;
        }
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            float q = 0.f;
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                const int c = 256 * k + 4 * lane;
                if (c < dim) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float d = x[i][k][j] - mean[i];
                        q += d * d;
                    }
                }
            }
            rstd[i] = __builtin_amdgcn_rsqf(wave_sum(q) * inv_dim + eps);
        }
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            const int64_t r = r0 + i;
            if (r >= rows) break;
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                const int c = 256 * k + 4 * lane;
                if (c < dim) {
                    float y[4];
                    Philox4 u{{0u, 0u, 0u, 0u}};
                    if (p > 0.f) u = philox4(seed, (uint64_t)r, (uint32_t)(c >> 2));
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        y[j] = (x[i][k][j] - mean[i]) * rstd[i] * gm[k][j] + bt[k][j];
                        if (p > 0.f) y[j] = u.w[j] >= thr ? y[j] * scale : 0.f;
                    }
                    store4(out + r * ldo + c, y);
                }
            }
            if (lane == 0 && mean_out) {
                mean_out[r] = mean[i];
                rstd_out[r] = rstd[i];
            }
        }
    }
}

// dz from dout (see the header); per-work-group dgamma / dbeta partials.
// ROWS rows in flight per wave, as in the forward.  The dropout mask is
// recomputed from Philox: as fast here as reading a stored bit mask, which
// would cost the forward its stores.
template <typename GT, typename ZT, int STEPS, int ROWS>
__global__ __launch_bounds__(kBlk) void act_norm_dropout_bwd_kernel(
    const GT* __restrict__ g, int64_t ldg, const ZT* __restrict__ z, int64_t ldz, int64_t rows, int dim, int act,
    const float* __restrict__ mean_in, const float* __restrict__ rstd_in, const float* __restrict__ gamma, float p,
    uint64_t seed, const uint64_t* __restrict__ seed_dev, ZT* __restrict__ dz, int64_t lddz,
    float* __restrict__ part_g, float* __restrict__ part_b) {
    __shared__ float red[2][kRowsPerBlock][STEPS * 256];
    if (seed_dev) seed = *seed_dev;
    const int lane = threadIdx.x & 63;
    // wave-uniform row index: mean, rstd and the mask words go through scalar loads
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t thr = keep_threshold(p);
    const float scale = p > 0.f ? 1.0f / (1.0f - p) : 1.0f;
    const float inv_dim = 1.0f / (float)dim;
    float ag[STEPS][4], ab[STEPS][4], gm[STEPS][4];
#pragma unroll
    for (int k = 0; k < STEPS; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ag[k][j] = ab[k][j] = 0.f;
            const int c = 256 * k + 4 * lane + j;
            gm[k][j] = c < dim ? gamma[c] : 0.f;
        }
    const int64_t stride = (int64_t)gridDim.x * kRowsPerBlock * ROWS;
    // the next iteration's rows are loaded while this one is computed
    typename Raw4<GT>::V rg[ROWS][STEPS];
    typename Raw4<ZT>::V rz[ROWS][STEPS];
    auto fetch = [&](int64_t rb) {
#pragma unroll
        for (int i = 0; i < ROWS; ++i)
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                const int c = 256 * k + 4 * lane;
                if (rb + i < rows && c < dim) {
                    rg[i][k] = load_raw4(g + (rb + i) * ldg + c);
                    rz[i][k] = load_raw4(z + (rb + i) * ldz + c);
                } else {
                    rg[i][k] = typename Raw4<GT>::V{};
                    rz[i][k] = typename Raw4<ZT>::V{};
                }
            }
    };
    int64_t r0 = ((int64_t)blockIdx.x * kRowsPerBlock + wave) * ROWS;
    if (r0 < rows) fetch(r0);
    for (; r0 < rows; r0 += stride) {
        float gv[ROWS][STEPS][4], zz[ROWS][STEPS][4];
#pragma unroll
        for (int i = 0; i < ROWS; ++i)
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                cvt4<GT>(rg[i][k], gv[i][k]);
                cvt4<ZT>(rz[i][k], zz[i][k]);
            }
        if (r0 + stride < rows) fetch(r0 + stride);
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            const int64_t r = r0 + i;
            if (r >= rows) break;
            const float mean = mean_in[r], rstd = rstd_in[r];
            float xh[STEPS][4], dxh[STEPS][4];
            float sa = 0.f, sb = 0.f;
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                const int c = 256 * k + 4 * lane;
                bool keep[4] = {true, true, true, true};
                if (p > 0.f) {
                    Philox4 u{{0u, 0u, 0u, 0u}};
                    if (c < dim) u = philox4(seed, (uint64_t)r, (uint32_t)(c >> 2));
#pragma unroll
                    for (int j = 0; j < 4; ++j) keep[j] = u.w[j] >= thr;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float x = zz[i][k][j];
                    if (act == 1) x = x < 0.f ? 0.f : x;
                    xh[k][j] = c < dim ? (x - mean) * rstd : 0.f;
                    float g1 = gv[i][k][j];
                    if (p > 0.f) g1 = keep[j] ? g1 * scale : 0.f;
                    ag[k][j] += g1 * xh[k][j];
                    ab[k][j] += g1;
                    dxh[k][j] = g1 * gm[k][j];
                    sa += dxh[k][j];
                    sb += dxh[k][j] * xh[k][j];
                }
            }
            const float a = wave_sum(sa) * inv_dim;
            const float b = wave_sum(sb) * inv_dim;
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                const int c = 256 * k + 4 * lane;
                if (c < dim) {
                    float d[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        d[j] = rstd * (dxh[k][j] - a - xh[k][j] * b);
                        if (act == 1 && zz[i][k][j] <= 0.f) d[j] = 0.f;  // threshold_backward on the result
                    }
                    store4(dz + r * lddz + c, d);
                }
            }
        }
    }
    // fixed-order reduction of the 4 waves, then one partial row per work-group
#pragma unroll
    for (int k = 0; k < STEPS; ++k) {
        const int c = 256 * k + 4 * lane;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            red[0][wave][c + j] = ag[k][j];
            red[1][wave][c + j] = ab[k][j];
        }
    }
    __syncthreads();
    for (int c = threadIdx.x; c < dim; c += kBlk) {
        float sg = 0.f, sbeta = 0.f;
#pragma unroll
        for (int w = 0; w < kRowsPerBlock; ++w) {
            sg += red[0][w][c];
            sbeta += red[1][w][c];
        }
        part_g[(int64_t)blockIdx.x * dim + c] = sg;
        part_b[(int64_t)blockIdx.x * dim + c] = sbeta;
    }
}

// out[c] = sum over parts of part[k][c]: 16 waves per 64 columns, wave w
// adding parts w, w+16, ... in order, then the 16 wave sums in order.
__global__ __launch_bounds__(1024) void column_sum_kernel(const float* __restrict__ part, int64_t nparts, int dim,
                                                          float* __restrict__ out) {
    __shared__ float red[16][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lane;
    float s = 0.f;
    if (c < dim) {
#pragma unroll 8
        for (int64_t k = wave; k < nparts; k += 16) s += part[k * dim + c];
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && c < dim) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < 16; ++w) t += red[w][lane];
        out[c] = t;
    }
}

// Upper bound of the backward's work-groups (and of its partial rows).
constexpr int64_t kMaxBwdBlocks = 4096;
int64_t bwd_blocks(int64_t rows) {
    int64_t b = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    if (b > kMaxBwdBlocks) b = kMaxBwdBlocks;
    return b < 1 ? 1 : b;
}

// Work-groups of `kernel` that fit on the device at once (all resident,
// equal shares of the rows, no second round of a few groups), at most cap.
template <typename K>
int64_t resident_blocks(K kernel, int64_t cap) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, kBlk, 0) != hipSuccess || cus <= 0 || per <= 0)
        return cap;
    const int64_t r = (int64_t)cus * per;
    return r < cap ? r : cap;
}

// ---------------------------------------------------------------------------
// cross-entropy
// ---------------------------------------------------------------------------
constexpr int64_t kIgnore = -100;

struct CeAcc {
    double loss;
    long long correct;
    long long valid;
    int bad;
};

// Whether (v, i) replaces the running (m, a) of an argmax: torch.argmax
// treats NaN as the maximum and returns the first index among equal maxima.
__device__ __forceinline__ bool argmax_better(float v, int i, float m, int a) {
    const bool vn = v != v, mn = m != m;
    if (vn) return !mn || i < a;
    if (mn) return false;
    return v > m || (v == m && i < a);
}

template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int d = LPR / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
    return v;
}

template <int LPR>
__device__ __forceinline__ double group_sum_d(double v) {
#pragma unroll
    for (int d = LPR / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
    return v;
}

// LPR lanes per selected row (16 for up to 64 classes: 4 rows per wave;
// 64 otherwise): lse, the label term, argmax (first index of the maximum,
// as torch.argmax).  Block partials of (loss, hits, valid rows, bad input).
template <typename T, int LPR>
__global__ __launch_bounds__(kBlk) void ce_fwd_kernel(const T* __restrict__ logits, int64_t ld, int64_t total_rows,
                                                      int classes, const int64_t* __restrict__ rows,
                                                      const int64_t* __restrict__ labels, int64_t n,
                                                      float* __restrict__ lse_out, double* __restrict__ part_loss,
                                                      long long* __restrict__ part_cnt) {
    constexpr int GPW = kWave / LPR;  // rows per wave
    __shared__ double sl[kRowsPerBlock];
    __shared__ long long sc[kRowsPerBlock], sv[kRowsPerBlock], sbad[kRowsPerBlock];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane % LPR;
    const int grp = lane / LPR;
    double wl = 0.0;
    long long wc = 0, wv = 0, wbad = 0;
    const int64_t stride = (int64_t)gridDim.x * kRowsPerBlock * GPW;
    for (int64_t i0 = ((int64_t)blockIdx.x * kRowsPerBlock + wave) * GPW; i0 < n; i0 += stride) {
        const int64_t i = i0 + grp;
        const bool live = i < n;
        const int64_t row = live ? (rows ? rows[i] : i) : 0;
        const int64_t lab = live ? labels[i] : kIgnore;
        const bool row_ok = live && row >= 0 && row < total_rows;
        const T* x = logits + (row_ok ? row : 0) * ld;
        float m = -INFINITY;
        int arg = 0x7fffffff;
        if (row_ok)
            for (int c = sub; c < classes; c += LPR) {
                const float v = to_float(x[c]);
                if (argmax_better(v, c, m, arg)) {
                    m = v;
                    arg = c;
                }
            }
#pragma unroll
        for (int d = LPR / 2; d > 0; d >>= 1) {
            const float om = __shfl_xor(m, d, kWave);
            const int oa = __shfl_xor(arg, d, kWave);
            if (argmax_better(om, oa, m, arg)) {
                m = om;
                arg = oa;
            }
        }
        float s = 0.f;
        if (row_ok)
            for (int c = sub; c < classes; c += LPR) s += expf(to_float(x[c]) - m);
        s = group_sum<LPR>(s);
        const float lse = m + logf(s);
        if (sub == 0 && live) {
            if (!row_ok) {
                wbad = 1;
            } else {
                lse_out[i] = lse;
                if (lab != kIgnore) {
                    if (lab < 0 || lab >= classes) {
                        wbad = 1;
                    } else {
                        wl += (double)(lse - to_float(x[lab]));
                        wv += 1;
                        wc += (arg == lab) ? 1 : 0;
                    }
                }
            }
        }
    }
    // the group leaders' sums, added over the wave (fixed order of the xor tree)
    wl = group_sum_d<kWave>(wl);
    wc = (long long)group_sum_d<kWave>((double)wc);
    wv = (long long)group_sum_d<kWave>((double)wv);
    wbad = (long long)group_sum_d<kWave>((double)wbad);
    if (lane == 0) {
        sl[wave] = wl;
        sc[wave] = wc;
        sv[wave] = wv;
        sbad[wave] = wbad ? 1 : 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double L = 0.0;
        long long C = 0, V = 0, B = 0;
        for (int w = 0; w < kRowsPerBlock; ++w) {
            L += sl[w];
            C += sc[w];
            V += sv[w];
            B |= sbad[w];
        }
        part_loss[blockIdx.x] = L;
        part_cnt[3 * blockIdx.x] = C;
        part_cnt[3 * blockIdx.x + 1] = V;
        part_cnt[3 * blockIdx.x + 2] = B;
    }
}

// loss = sum / valid (NaN when no row counts or a label is out of range:
// torch asserts there), correct = hits, valid = counted rows.  One
// work-group: thread t adds parts t, t+256, ... in order, then thread 0 the
// 256 sums in order (deterministic).
__global__ __launch_bounds__(256) void ce_finish_kernel(const double* __restrict__ part_loss,
                                                        const long long* __restrict__ part_cnt, int64_t nparts,
                                                        float* __restrict__ loss, int64_t* __restrict__ counts) {
    __shared__ double sl[256];
    __shared__ long long sc[256], sv[256], sb[256];
    double L = 0.0;
    long long C = 0, V = 0, B = 0;
    for (int64_t k = threadIdx.x; k < nparts; k += 256) {
        L += part_loss[k];
        C += part_cnt[3 * k];
        V += part_cnt[3 * k + 1];
        B |= part_cnt[3 * k + 2];
    }
    sl[threadIdx.x] = L;
    sc[threadIdx.x] = C;
    sv[threadIdx.x] = V;
    sb[threadIdx.x] = B;
    __syncthreads();
    if (threadIdx.x != 0) return;
    L = 0.0;
    C = V = B = 0;
    for (int t = 0; t < 256; ++t) {
        L += sl[t];
        C += sc[t];
        V += sv[t];
        B |= sb[t];
    }
    loss[0] = (B || V == 0) ? __int_as_float(0x7fc00000) : (float)(L / (double)V);
    counts[0] = C;
    counts[1] = V;
    counts[2] = B;
}

// grad[row][c] = (softmax - onehot) * dloss / valid for counted rows, 0 for
// ignored ones; other rows of grad are left alone (the caller zero-fills).
template <typename T, typename GT, int LPR>
__global__ __launch_bounds__(kBlk) void ce_bwd_kernel(const T* __restrict__ logits, int64_t ld, int64_t total_rows,
                                                      int classes, const int64_t* __restrict__ rows,
                                                      const int64_t* __restrict__ labels, int64_t n,
                                                      const float* __restrict__ lse, const float* __restrict__ dloss,
                                                      const int64_t* __restrict__ counts, GT* __restrict__ grad,
                                                      int64_t ldg) {
    constexpr int GPW = kWave / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane % LPR;
    const int64_t valid = counts[1];
    const float scale = valid > 0 ? dloss[0] / (float)valid : 0.f;
    const int64_t stride = (int64_t)gridDim.x * kRowsPerBlock * GPW;
    for (int64_t i = ((int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) * GPW + lane / LPR; i < n;
         i += stride) {
        const int64_t row = rows ? rows[i] : i;
        if (row < 0 || row >= total_rows) continue;
        const int64_t lab = labels[i];
        const bool counted = lab != kIgnore && lab >= 0 && lab < classes;
        const float l = lse[i];
        for (int c = sub; c < classes; c += LPR) {
            float v = 0.f;
            if (counted) v = (expf(to_float(logits[row * ld + c]) - l) - (c == lab ? 1.f : 0.f)) * scale;
            grad[row * ldg + c] = from_float<GT>(v);
        }
    }
}

int64_t ce_blocks(int64_t n) {
    int64_t b = (n + kRowsPerBlock - 1) / kRowsPerBlock;
    if (b > 4096) b = 4096;
    return b < 1 ? 1 : b;
}

}  // namespace
}  // namespace grws

using namespace grws;

extern "C" size_t grws_act_norm_dropout_bwd_workspace_bytes(int64_t rows, int64_t dim) {
    if (rows < 0 || dim < 0) return 0;
    Sizer s;
    s.take<float>((size_t)bwd_blocks(rows) * (size_t)dim);
    s.take<float>((size_t)bwd_blocks(rows) * (size_t)dim);
    return s.used;
}

#define GRWS_DISPATCH2(DT_A, DT_B, MACRO)                                                          \
    do {                                                                                           \
        if ((DT_A) == GRWS_F32) {                                                                  \
            if ((DT_B) == GRWS_F32) MACRO(float, float);                                           \
            else if ((DT_B) == GRWS_F16) MACRO(float, _Float16);                                   \
            else MACRO(float, __hip_bfloat16);                                                     \
        } else if ((DT_A) == GRWS_F16) {                                                           \
            if ((DT_B) == GRWS_F32) MACRO(_Float16, float);                                        \
            else if ((DT_B) == GRWS_F16) MACRO(_Float16, _Float16);                                \
            else MACRO(_Float16, __hip_bfloat16);                                                  \
        } else {                                                                                   \
            if ((DT_B) == GRWS_F32) MACRO(__hip_bfloat16, float);                                  \
            else if ((DT_B) == GRWS_F16) MACRO(__hip_bfloat16, _Float16);                          \
            else MACRO(__hip_bfloat16, __hip_bfloat16);                                            \
        }                                                                                          \
    } while (0)

static int check_rowwise(int32_t a_dt, int32_t b_dt, int64_t rows, int64_t dim, int64_t lda, int64_t ldb,
                         const void* a, const void* b) {
    for (int32_t dt : {a_dt, b_dt})
        if (dt != GRWS_F32 && dt != GRWS_F16 && dt != GRWS_BF16)
            return set_error(GRWS_E_DTYPE, "act_norm_dropout: unsupported dtype %d", dt);
    GRWS_CHECK_ARG(rows >= 0, "act_norm_dropout: negative rows");
    GRWS_CHECK_ARG(dim > 0 && dim <= 1024 && dim % 4 == 0, "act_norm_dropout: dim must be 4..1024, a multiple of 4");
    GRWS_CHECK_ARG(lda >= dim && ldb >= dim && lda % 4 == 0 && ldb % 4 == 0,
                   "act_norm_dropout: leading dimensions must be >= dim and multiples of 4");
    GRWS_CHECK_ARG((reinterpret_cast<uintptr_t>(a) % 8) == 0 && (reinterpret_cast<uintptr_t>(b) % 8) == 0,
                   "act_norm_dropout: rows must be 8-byte aligned");
    return GRWS_OK;
}

extern "C" int grws_act_norm_dropout_fwd(const void* z, int32_t z_dtype, int64_t ldz, int64_t rows, int64_t dim,
                                         int32_t act, const float* gamma, const float* beta, float eps, float p,
                                         uint64_t seed, const uint64_t* seed_dev, void* out, int32_t out_dtype,
                                         int64_t ldo, float* mean, float* rstd, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(act == 0 || act == 1, "act_norm_dropout: act must be 0 (none) or 1 (relu)");
    GRWS_CHECK_ARG(p >= 0.f && p < 1.f, "act_norm_dropout: p must be in [0, 1)");
    GRWS_CHECK_ARG((mean == nullptr) == (rstd == nullptr), "act_norm_dropout: mean and rstd go together");
    if (rows == 0) return GRWS_OK;
    GRWS_CHECK_ARG(z && out && gamma && beta, "act_norm_dropout: null pointer");
    GRWS_TRY(check_rowwise(z_dtype, out_dtype, rows, dim, ldz, ldo, z, out));
    const int steps = (int)((dim + 255) / 256);
    const int rpw = steps == 1 ? 4 : (steps == 2 ? 2 : 1);  // rows in flight per wave
    // a few passes per wave (its next rows load during the current ones):
    // measured faster than one pass per wave or a resident-only grid
    int64_t blocks = (rows + kRowsPerBlock * rpw - 1) / (kRowsPerBlock * rpw);
    if (blocks > 65536) blocks = 65536;
#define GRWS_ANDF_SR(ZT, OT, S, R)                                                                              \
    hipLaunchKernelGGL((act_norm_dropout_fwd_kernel<ZT, OT, S, R>), dim3((unsigned)blocks), dim3(kBlk), 0, stream, \
                       static_cast<const ZT*>(z), ldz, rows, (int)dim, (int)act, gamma, beta, eps, p, seed,       \
                       seed_dev, static_cast<OT*>(out), ldo, mean, rstd)
#define GRWS_ANDF(ZT, OT)                              \
    do {                                               \
        if (steps == 1) GRWS_ANDF_SR(ZT, OT, 1, 4);    \
        else if (steps == 2) GRWS_ANDF_SR(ZT, OT, 2, 2); \
        else if (steps == 3) GRWS_ANDF_SR(ZT, OT, 3, 1); \
        else GRWS_ANDF_SR(ZT, OT, 4, 1);               \
    } while (0)
    GRWS_DISPATCH2(z_dtype, out_dtype, GRWS_ANDF);
#undef GRWS_ANDF
#undef GRWS_ANDF_SR
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

extern "C" int grws_act_norm_dropout_bwd(const void* dout, int32_t dout_dtype, int64_t ldg, const void* z,
                                         int32_t z_dtype, int64_t ldz, int64_t rows, int64_t dim, int32_t act,
                                         const float* mean, const float* rstd, const float* gamma, float p,
                                         uint64_t seed, const uint64_t* seed_dev, void* dz, int64_t lddz,
                                         float* dgamma, float* dbeta,
                                         void* workspace, size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(act == 0 || act == 1, "act_norm_dropout: act must be 0 (none) or 1 (relu)");
    GRWS_CHECK_ARG(p >= 0.f && p < 1.f, "act_norm_dropout: p must be in [0, 1)");
    GRWS_CHECK_ARG(dgamma && dbeta, "act_norm_dropout: null dgamma/dbeta");
    GRWS_CHECK_ARG(dim > 0 && dim <= 1024 && dim % 4 == 0, "act_norm_dropout: dim must be 4..1024, a multiple of 4");
    if (rows == 0) {
        GRWS_TRY(fill_bytes_zero(dgamma, (size_t)dim * 4, stream));
        GRWS_TRY(fill_bytes_zero(dbeta, (size_t)dim * 4, stream));
        return GRWS_OK;
    }
    GRWS_CHECK_ARG(dout && z && mean && rstd && gamma && dz, "act_norm_dropout: null pointer");
    GRWS_TRY(check_rowwise(dout_dtype, z_dtype, rows, dim, ldg, ldz, dout, z));
    GRWS_CHECK_ARG(lddz >= dim && lddz % 4 == 0 && (reinterpret_cast<uintptr_t>(dz) % 8) == 0,
                   "act_norm_dropout: bad dz layout");
    const int64_t blocks = bwd_blocks(rows);
    int64_t nb = blocks;  // launched work-groups: the resident count, at most `blocks`
    Carver cv(workspace, workspace_bytes);
    float* pg = cv.take<float>((size_t)blocks * (size_t)dim);
    float* pb = cv.take<float>((size_t)blocks * (size_t)dim);
    if (!cv.ok)
        return set_error(GRWS_E_CAPACITY, "act_norm_dropout: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const int steps = (int)((dim + 255) / 256);
#define GRWS_ANDB_SR(GT, ZT, S, R)                                                                              \
    do {                                                                                                         \
        nb = resident_blocks(act_norm_dropout_bwd_kernel<GT, ZT, S, R>, blocks);                                 \
        hipLaunchKernelGGL((act_norm_dropout_bwd_kernel<GT, ZT, S, R>), dim3((unsigned)nb), dim3(kBlk), 0, stream, \
                           static_cast<const GT*>(dout), ldg, static_cast<const ZT*>(z), ldz, rows, (int)dim,      \
                           (int)act, mean, rstd, gamma, p, seed, seed_dev, static_cast<ZT*>(dz), lddz, pg, pb);              \
    } while (0)
#define GRWS_ANDB(GT, ZT)                              \
    do {                                               \
        if (steps == 1) GRWS_ANDB_SR(GT, ZT, 1, 4);    \
        else if (steps == 2) GRWS_ANDB_SR(GT, ZT, 2, 2); \
        else if (steps == 3) GRWS_ANDB_SR(GT, ZT, 3, 1); \
        else GRWS_ANDB_SR(GT, ZT, 4, 1);               \
    } while (0)
    GRWS_DISPATCH2(dout_dtype, z_dtype, GRWS_ANDB);
#undef GRWS_ANDB
#undef GRWS_ANDB_SR
    GRWS_LAUNCH_CHECK();
    const unsigned cb = (unsigned)((dim + 63) / 64);
    hipLaunchKernelGGL(column_sum_kernel, dim3(cb), dim3(1024), 0, stream, pg, nb, (int)dim, dgamma);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(column_sum_kernel, dim3(cb), dim3(1024), 0, stream, pb, nb, (int)dim, dbeta);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

extern "C" size_t grws_cross_entropy_workspace_bytes(int64_t n) {
    if (n < 0) return 0;
    Sizer s;
    s.take<double>((size_t)ce_blocks(n));
    s.take<long long>(3 * (size_t)ce_blocks(n));
    return s.used;
}

extern "C" int grws_cross_entropy_fwd(const void* logits, int32_t dtype, int64_t ld, int64_t total_rows,
                                      int64_t classes, const int64_t* rows, const int64_t* labels, int64_t n,
                                      float* lse_out, float* loss_out, int64_t* counts_out, void* workspace,
                                      size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    if (dtype != GRWS_F32 && dtype != GRWS_F16 && dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "cross_entropy: unsupported dtype %d", dtype);
    GRWS_CHECK_ARG(classes > 0 && classes <= INT32_MAX && ld >= classes && n >= 0 && total_rows >= 0,
                   "cross_entropy: bad sizes");
    GRWS_CHECK_ARG(loss_out && counts_out, "cross_entropy: null output");
    if (n > 0) GRWS_CHECK_ARG(logits && labels && lse_out, "cross_entropy: null pointer");
    const int64_t blocks = ce_blocks(n);
    Carver cv(workspace, workspace_bytes);
    double* pl = cv.take<double>((size_t)blocks);
    long long* pc = cv.take<long long>(3 * (size_t)blocks);
    if (!cv.ok)
        return set_error(GRWS_E_CAPACITY, "cross_entropy: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const bool narrow = classes <= 64;
#define GRWS_CEF_L(T, L)                                                                                       \
    hipLaunchKernelGGL((ce_fwd_kernel<T, L>), dim3((unsigned)blocks), dim3(kBlk), 0, stream,                   \
                       static_cast<const T*>(logits), ld, total_rows, (int)classes, rows, labels, n, lse_out, pl, pc)
#define GRWS_CEF(T)                                \
    do {                                           \
        if (narrow) GRWS_CEF_L(T, 16);             \
        else GRWS_CEF_L(T, 64);                    \
    } while (0)
    if (dtype == GRWS_F32) GRWS_CEF(float);
    else if (dtype == GRWS_F16) GRWS_CEF(_Float16);
    else GRWS_CEF(__hip_bfloat16);
#undef GRWS_CEF
#undef GRWS_CEF_L
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(ce_finish_kernel, dim3(1), dim3(256), 0, stream, pl, pc, blocks, loss_out, counts_out);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

extern "C" int grws_cross_entropy_bwd(const void* logits, int32_t dtype, int64_t ld, int64_t total_rows,
                                      int64_t classes, const int64_t* rows, const int64_t* labels, int64_t n,
                                      const float* lse, const float* dloss, const int64_t* counts, void* grad,
                                      int32_t grad_dtype, int64_t ldg, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    if (dtype != GRWS_F32 && dtype != GRWS_F16 && dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "cross_entropy: unsupported dtype %d", dtype);
    if (grad_dtype != GRWS_F32 && grad_dtype != GRWS_F16 && grad_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "cross_entropy: unsupported grad dtype %d", grad_dtype);
    GRWS_CHECK_ARG(classes > 0 && classes <= INT32_MAX && ld >= classes && ldg >= classes && n >= 0,
                   "cross_entropy: bad sizes");
    if (n == 0) return GRWS_OK;
    GRWS_CHECK_ARG(logits && labels && lse && dloss && counts && grad, "cross_entropy: null pointer");
    const int64_t blocks = ce_blocks(n);
    const bool narrow = classes <= 64;
#define GRWS_CEB_L(T, GT, L)                                                                                   \
    hipLaunchKernelGGL((ce_bwd_kernel<T, GT, L>), dim3((unsigned)blocks), dim3(kBlk), 0, stream,               \
                       static_cast<const T*>(logits), ld, total_rows, (int)classes, rows, labels, n, lse, dloss,  \
                       counts, static_cast<GT*>(grad), ldg)
#define GRWS_CEB(T, GT)                            \
    do {                                           \
        if (narrow) GRWS_CEB_L(T, GT, 16);         \
        else GRWS_CEB_L(T, GT, 64);                \
    } while (0)
    GRWS_DISPATCH2(dtype, grad_dtype, GRWS_CEB);
#undef GRWS_CEB
#undef GRWS_CEB_L
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}
