// Weight gradient C[M x N] = A^T B for tall, skinny operands (gfx950).
//
// The backward of the reference's graph convolution computes
// grad_weight = features^T @ grad_input_aggr (layers/layer.py:61-92) and,
// through autograd, the self path's weight gradient the same way
// (layer.py:171-175): K = the node count (10^5..10^6), M and N = the layer
// widths (<= a few hundred).  A library GEMM tiles the small M x N output
// into a handful of work-groups, so most of the chip idles while each
// streams all of K.  Here K is split instead:
//   * work-group (M-tile of 128, N-tile of 128, K-chunk): 4 wave64s, each a
//     64 x 64 block of the output as 4 x 4 v_mfma_f32_16x16x16 tiles;
//   * per step, 32 rows of A and B (128 columns each) are loaded with
//     16-byte coalesced loads into two alternating LDS stages; the next
//     step's rows are loaded into registers while the current stage is
//     multiplied;
//   * both MFMA operands are columns of the staged rows (A^T needs A's
//     columns, 4 consecutive k per lane), read with gfx950's transposing
//     LDS read: one ds_read_b64_tr_b16 per operand per 16 k;
//   * every chunk writes an fp32 partial; a second kernel adds the chunks
//     in order (deterministic, no atomics) and writes C.
// A and B are each read once per N-tile / M-tile of the other operand; the
// work-groups of one K-chunk (all its output tiles) are dealt to the same
// XCD one after another, so the second read of a chunk's rows hits that
// XCD's L2 instead of going out to memory again.
#include "grws_internal.h"

namespace grws {
namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 tr_v4f16_t;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 tr_v4bf16_t;
typedef __attribute__((address_space(3))) tr_v4f16_t lds_v4f16_t;
typedef __attribute__((address_space(3))) tr_v4bf16_t lds_v4bf16_t;

constexpr int kT = 128;       // output tile edge
constexpr int kStep = 32;     // K rows per LDS stage
constexpr int kPitch = kT + 8;  // LDS row pitch (elements)
constexpr int kMaxChunks = 512;
constexpr int64_t kMinChunkRows = 1024;

// Column block of 16 (columns c0..c0+15) of rows k..k+15 of a staged
// operand as the MFMA's 16x16x16 operand: lane (g, i) gets rows 4g..4g+3 of
// column c0 + i.  The 16 lanes of a group read 4 halves each at row
// 4g + (lane%16)/4, column c0 + 4 (lane%4); the transposing read hands
// lane i column i of the group's 4 rows.
template <int DT>
__device__ __forceinline__ short4_t lds_col_frag(const uint16_t* stage, int k, int c0, int lane) {
    const uint16_t* p = stage + (k + 4 * (lane >> 4) + ((lane & 15) >> 2)) * kPitch + c0 + 4 * (lane & 3);
    if constexpr (DT == GRWS_F16) {
        return __builtin_bit_cast(short4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                                (lds_v4f16_t*)(__attribute__((address_space(3))) void*)p));
    } else {
        return __builtin_bit_cast(short4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                                                (lds_v4bf16_t*)(__attribute__((address_space(3))) void*)p));
    }
}

template <int DT>
__global__ __launch_bounds__(256) void gemm_tn_partial_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                              const uint16_t* __restrict__ B, int64_t ldb,
                                                              int64_t K, int M, int N, int64_t kc,
                                                              int64_t nchunks, float* __restrict__ partials) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][kStep * kPitch];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][kStep * kPitch];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    // work-groups are dealt round-robin to the 8 XCDs: block b runs on XCD
    // b % 8.  Slot b / 8 of an XCD walks the output tiles of chunk
    // (slot / tiles) * 8 + xcd, so a chunk's tiles share one L2.
    const int tiles_m = (M + kT - 1) / kT;
    const int tiles = tiles_m * ((N + kT - 1) / kT);
    const int64_t blk = blockIdx.x;
    const int64_t slot = blk >> 3;
    const int t = (int)(slot % tiles);
    const int64_t chunk = (slot / tiles) * 8 + (blk & 7);
    if (chunk >= nchunks) return;  // uniform over the work-group
    const int i0 = (t % tiles_m) * kT;
    const int j0 = (t / tiles_m) * kT;
    const int64_t kb = chunk * kc;
    const int64_t ke = kb + kc < K ? kb + kc : K;
    const int wm = (wave & 1) * 64;
    const int wn = (wave >> 1) * 64;
    const int fr = lane & 15;        // output column within a 16 x 16 tile
    const int fk = (lane >> 4) * 4;  // first output row of the lane within a tile

    float4_t acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    // staging geometry: 32 rows x 128 columns = 512 loads of 8 elements,
    // two per thread for each operand
    u32x4_t ra[2], rb[2];
    auto fetch = [&](int64_t k0) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int e = (tid + 256 * q) * 8;
            const int r = e / kT, c = e % kT;
            const int64_t k = k0 + r;
            const bool okr = k < ke;
            ra[q] = u32x4_t{0u, 0u, 0u, 0u};
            rb[q] = u32x4_t{0u, 0u, 0u, 0u};
            if (okr && i0 + c < M) ra[q] = *reinterpret_cast<const u32x4_t*>(A + k * lda + i0 + c);
            if (okr && j0 + c < N) rb[q] = *reinterpret_cast<const u32x4_t*>(B + k * ldb + j0 + c);
        }
    };
    int buf = 0;
    if (kb < ke) fetch(kb);
    for (int64_t k0 = kb; k0 < ke; k0 += kStep) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int e = (tid + 256 * q) * 8;
            const int r = e / kT, c = e % kT;
            *reinterpret_cast<u32x4_t*>(&sA[buf][r * kPitch + c]) = ra[q];
            *reinterpret_cast<u32x4_t*>(&sB[buf][r * kPitch + c]) = rb[q];
        }
        __syncthreads();  // the stage is written; the other stage's readers are done
        if (k0 + kStep < ke) fetch(k0 + kStep);
#pragma unroll
        for (int ks = 0; ks < kStep; ks += 16) {
            short4_t af[4], bf[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                af[t] = lds_col_frag<DT>(sA[buf], ks, wm + 16 * t, lane);
                bf[t] = lds_col_frag<DT>(sB[buf], ks, wn + 16 * t, lane);
            }
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    if constexpr (DT == GRWS_F16)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, af[a]),
                                                                          __builtin_bit_cast(half4_t, bf[b]),
                                                                          acc[a][b], 0, 0, 0);
                    else
                        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(af[a], bf[b], acc[a][b], 0, 0, 0);
                }
        }
        buf ^= 1;
    }
    // D layout: lane l, element e -> row 4*(l/16)+e, column l%16 of the tile
    float* P = partials + chunk * (int64_t)M * N;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int j = j0 + wn + 16 * b + fr;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = i0 + wm + 16 * a + fk + e;
                if (i < M && j < N) P[(int64_t)i * N + j] = acc[a][b][e];
            }
        }
}

// C[i][j] = sum over chunks.  A work-group of 16 waves covers 64
// consecutive outputs; wave w adds chunks w, w+16, ... in order (coalesced
// 256-byte rows), then wave 0 adds the 16 wave sums in order: a fixed order
// (deterministic), with 16 waves' loads in flight per output group.
template <int OT>
__global__ __launch_bounds__(1024) void gemm_tn_reduce_kernel(const float* __restrict__ partials, int64_t nchunks,
                                                              int M, int N, void* c, int64_t ldc) {
    __shared__ float red[16][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t mn = (int64_t)M * N;
    const int64_t idx = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.f;
    if (idx < mn) {
#pragma unroll 8
        for (int64_t ch = wave; ch < nchunks; ch += 16) s += partials[ch * mn + idx];
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave != 0 || idx >= mn) return;
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) t += red[w][lane];
    const int64_t i = idx / N, j = idx % N;
    if constexpr (OT == GRWS_F32) {
        static_cast<float*>(c)[i * ldc + j] = t;
    } else if constexpr (OT == GRWS_F16) {
        static_cast<_Float16*>(c)[i * ldc + j] = (_Float16)t;
    } else {
        static_cast<__hip_bfloat16*>(c)[i * ldc + j] = __float2bfloat16(t);
    }
}

// K-chunks: of kMinChunkRows rows, or, when that leaves fewer than
// kMinBlocks work-groups (a mini-batch's few thousand rows), of as few as
// kSmallChunkRows rows until there are kMinBlocks; at most kMaxChunks.
constexpr int64_t kSmallChunkRows = 256;
constexpr int64_t kMinBlocks = 256;

int64_t chunks_for(int64_t K, int64_t M, int64_t N) {
    const int64_t tiles = ((M + kT - 1) / kT) * ((N + kT - 1) / kT);
    int64_t n = (K + kMinChunkRows - 1) / kMinChunkRows;
    if (tiles > 0 && n * tiles < kMinBlocks) {
        const int64_t small = (K + kSmallChunkRows - 1) / kSmallChunkRows;
        const int64_t want = (kMinBlocks + tiles - 1) / tiles;
        n = small < want ? small : want;
    }
    if (n > kMaxChunks) n = kMaxChunks;
    return n < 1 ? 1 : n;
}

}  // namespace
}  // namespace grws

using namespace grws;

extern "C" size_t grws_gemm_tn_workspace_bytes(int64_t K, int64_t M, int64_t N) {
    if (K < 0 || M < 0 || N < 0) return 0;
    return (size_t)chunks_for(K, M, N) * (size_t)M * (size_t)N * sizeof(float);
}

extern "C" int grws_gemm_tn(const void* a, int64_t lda, const void* b, int64_t ldb, int32_t in_dtype, int64_t K,
                            int64_t M, int64_t N, void* c, int64_t ldc, int32_t out_dtype, void* workspace,
                            size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(K >= 0 && M >= 0 && N >= 0, "gemm_tn: negative size");
    GRWS_CHECK_ARG(M <= 65536 && N <= 65536, "gemm_tn: M and N must be at most 65536");
    if (in_dtype != GRWS_F16 && in_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "gemm_tn: inputs must be F16 or BF16 (got %d)", in_dtype);
    if (out_dtype != GRWS_F32 && out_dtype != in_dtype)
        return set_error(GRWS_E_DTYPE, "gemm_tn: output must be F32 or the input dtype");
    GRWS_CHECK_ARG(M % 8 == 0 && N % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0,
                   "gemm_tn: M, N, lda and ldb must be multiples of 8");
    GRWS_CHECK_ARG(lda >= M && ldb >= N && ldc >= N, "gemm_tn: leading dimensions too small");
    if (M == 0 || N == 0) return GRWS_OK;
    GRWS_CHECK_ARG(c != nullptr, "gemm_tn: null output");
    if (K > 0) {
        GRWS_CHECK_ARG(a && b, "gemm_tn: null input");
        GRWS_CHECK_ARG((reinterpret_cast<uintptr_t>(a) % 16) == 0 && (reinterpret_cast<uintptr_t>(b) % 16) == 0,
                       "gemm_tn: inputs must be 16-byte aligned");
    }
    const int64_t nch = K > 0 ? chunks_for(K, M, N) : 0;
    const size_t need = (size_t)nch * (size_t)M * (size_t)N * sizeof(float);
    if (nch > 0 && (!workspace || workspace_bytes < need))
        return set_error(GRWS_E_CAPACITY, "gemm_tn: workspace too small (%zu < %zu)", workspace_bytes, need);
    int64_t chunks = 0;  // K == 0: the reduction over no chunks writes zeros
    if (nch > 0) {
        const int64_t kc = ((K + nch - 1) / nch + kStep - 1) / kStep * kStep;
        chunks = (K + kc - 1) / kc;
        const int64_t tiles = ((M + kT - 1) / kT) * ((N + kT - 1) / kT);
        const int64_t blocks = (chunks + 7) / 8 * 8 * tiles;  // chunks padded to whole XCD rounds
        GRWS_CHECK_ARG(blocks <= INT32_MAX, "gemm_tn: too many work-groups");
        if (in_dtype == GRWS_F16)
            hipLaunchKernelGGL(gemm_tn_partial_kernel<GRWS_F16>, dim3((unsigned)blocks), dim3(256), 0, stream,
                               static_cast<const uint16_t*>(a), lda, static_cast<const uint16_t*>(b), ldb, K,
                               (int)M, (int)N, kc, chunks, static_cast<float*>(workspace));
        else
            hipLaunchKernelGGL(gemm_tn_partial_kernel<GRWS_BF16>, dim3((unsigned)blocks), dim3(256), 0, stream,
                               static_cast<const uint16_t*>(a), lda, static_cast<const uint16_t*>(b), ldb, K,
                               (int)M, (int)N, kc, chunks, static_cast<float*>(workspace));
        GRWS_LAUNCH_CHECK();
    }
    {
        const unsigned rg = (unsigned)((M * N + 63) / 64);
        switch (out_dtype) {
            case GRWS_F32:
                hipLaunchKernelGGL(gemm_tn_reduce_kernel<GRWS_F32>, dim3(rg), dim3(1024), 0, stream,
                                   static_cast<const float*>(workspace), chunks, (int)M, (int)N, c, ldc);
                break;
            case GRWS_F16:
                hipLaunchKernelGGL(gemm_tn_reduce_kernel<GRWS_F16>, dim3(rg), dim3(1024), 0, stream,
                                   static_cast<const float*>(workspace), chunks, (int)M, (int)N, c, ldc);
                break;
            default:
                hipLaunchKernelGGL(gemm_tn_reduce_kernel<GRWS_BF16>, dim3(rg), dim3(1024), 0, stream,
                                   static_cast<const float*>(workspace), chunks, (int)M, (int)N, c, ldc);
                break;
        }
        GRWS_LAUNCH_CHECK();
    }
    return GRWS_OK;
}
