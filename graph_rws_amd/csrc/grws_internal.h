// Internal helpers shared by the libgrws translation units (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>

#include <mutex>
#include <type_traits>

#include "grws_host.h"

namespace grws {

#define GRWS_HIP(call)                                                                   \
    do {                                                                                 \
        hipError_t e_ = (call);                                                          \
        if (e_ != hipSuccess)                                                            \
            return ::grws::set_error(GRWS_E_HIP, "%s:%d %s: %s", __FILE__, __LINE__, #call, \
                                     hipGetErrorString(e_));                             \
    } while (0)

#define GRWS_LAUNCH_CHECK()                                                              \
    do {                                                                                 \
        hipError_t e_ = hipGetLastError();                                               \
        if (e_ != hipSuccess)                                                            \
            return ::grws::set_error(GRWS_E_HIP, "%s:%d kernel launch: %s", __FILE__, __LINE__, \
                                     hipGetErrorString(e_));                             \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Carves aligned sub-buffers out of a caller workspace.
struct Carver {
    char* base;
    size_t cap;
    size_t used = 0;
    bool ok = true;
    Carver(void* b, size_t c) : base(static_cast<char*>(b)), cap(c) {}
    template <typename T>
    T* take(size_t n) {
        size_t off = align_up(used, 256);
        size_t bytes = align_up(n * sizeof(T), 256);
        if (off + bytes > cap || (base == nullptr && bytes > 0)) {
            ok = false;
            used = off + bytes;
            return nullptr;
        }
        used = off + bytes;
        return reinterpret_cast<T*>(base + off);
    }
};

// Size-only twin of Carver (for *_workspace_bytes queries).
struct Sizer {
    size_t used = 0;
    template <typename T>
    void take(size_t n) {
        used = align_up(used, 256) + align_up(n * sizeof(T), 256);
    }
};

// A second stream for work that would leave most of the GPU idle if it ran
// after the rest (a few long work-groups).  One such stream per device,
// created on first use with the default priority; each call forks from the
// caller's stream and joins back into it through events of its own, so
// concurrent calls stay ordered.  When the caller's stream belongs to another
// device than the current one, or the device index is out of range, the side
// work stays on the caller's stream.  So it does when the caller's stream is
// being captured (or its capture state cannot be read): a fork there would
// pull the shared stream into the caller's graph, and a call on another
// thread would then land in that graph.
constexpr int kSideDevices = 64;

inline int side_fork(hipStream_t main, hipStream_t* side) {
    *side = main;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(main, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return GRWS_OK;
    }
    if (cs != hipStreamCaptureStatusNone) return GRWS_OK;
    int dev = 0;
    GRWS_HIP(hipGetDevice(&dev));
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(main, &sdev) != hipSuccess) {
        (void)hipGetLastError();  // clears the failed query's error
        return GRWS_OK;
    }
    if (sdev != dev || dev < 0 || dev >= kSideDevices) return GRWS_OK;
    static std::mutex mu;
    static hipStream_t streams[kSideDevices] = {};
    hipStream_t s = nullptr;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (!streams[dev]) GRWS_HIP(hipStreamCreateWithFlags(&streams[dev], hipStreamNonBlocking));
        s = streams[dev];
    }
    hipEvent_t ev;
    GRWS_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    hipError_t e = hipEventRecord(ev, main);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, ev, 0);
    (void)hipEventDestroy(ev);
    GRWS_HIP(e);
    *side = s;
    return GRWS_OK;
}

inline int side_join(hipStream_t main, hipStream_t side) {
    if (side == main) return GRWS_OK;
    hipEvent_t ev;
    GRWS_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    hipError_t e = hipEventRecord(ev, side);
    if (e == hipSuccess) e = hipStreamWaitEvent(main, ev, 0);
    (void)hipEventDestroy(ev);
    GRWS_HIP(e);
    return GRWS_OK;
}

// A forked side stream that is joined back on every exit: an error return
// between the fork and the join must not leave side work running on a
// workspace the caller may free (and its allocator hand out again on the
// caller's stream).  join() reports the join's status; the destructor joins
// quietly (the first error's message stays), and when even the events fail
// it waits for the side stream.
struct SideStream {
    hipStream_t main, side;
    explicit SideStream(hipStream_t m) : main(m), side(m) {}
    SideStream(const SideStream&) = delete;
    SideStream& operator=(const SideStream&) = delete;
    int fork() { return side_fork(main, &side); }
    // fork onto a caller-owned stream `s` instead (a capture's own second
    // stream: under capture the event wait joins `s` into the capture, and
    // no other caller shares it); null keeps the work on `main`
    int fork_to(hipStream_t s) {
        if (s == nullptr || s == main) return GRWS_OK;
        int md = -1;
        hipDevice_t sd = -1;
        if (main == nullptr) {
            GRWS_HIP(hipGetDevice(&md));
        } else {
            hipDevice_t d = -1;
            GRWS_HIP(hipStreamGetDevice(main, &d));
            md = (int)d;
        }
        GRWS_HIP(hipStreamGetDevice(s, &sd));
        if (md != sd)
            return set_error(GRWS_E_INVALID, "side stream on device %d, the call's stream on device %d", (int)sd,
                             (int)md);
        hipEvent_t ev;
        GRWS_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        hipError_t e = hipEventRecord(ev, main);
        if (e == hipSuccess) e = hipStreamWaitEvent(s, ev, 0);
        (void)hipEventDestroy(ev);
        GRWS_HIP(e);
        side = s;
        return GRWS_OK;
    }
    int join() {
        const hipStream_t s = side;
        side = main;
        return side_join(main, s);
    }
    ~SideStream() {
        if (side == main) return;
        hipEvent_t ev;
        hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e == hipSuccess) {
            e = hipEventRecord(ev, side);
            if (e == hipSuccess) e = hipStreamWaitEvent(main, ev, 0);
            (void)hipEventDestroy(ev);
        }
        if (e != hipSuccess) (void)hipStreamSynchronize(side);
        (void)hipGetLastError();
    }
};

// ---------------------------------------------------------------------------
// device helpers (wave64)
// ---------------------------------------------------------------------------
constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t lanemask_lt() {
    int l = __lane_id();
    return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// Inclusive wave scan (sum) of a 64-bit value.
__device__ __forceinline__ int64_t wave_incl_scan(int64_t v) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        int64_t t = __shfl_up(v, d, kWave);
        if (__lane_id() >= d) v += t;
    }
    return v;
}

// Block-wide inclusive scan for blockDim.x == BLOCK (multiple of 64).
// `smem` needs BLOCK/64 + 1 int64 slots.  Returns inclusive prefix; *total
// receives the block sum.  Contains __syncthreads.
template <int BLOCK>
__device__ __forceinline__ int64_t block_incl_scan(int64_t v, int64_t* smem, int64_t* total) {
    constexpr int NW = BLOCK / kWave;
    const int w = threadIdx.x / kWave;
    int64_t inc = wave_incl_scan(v);
    if (__lane_id() == kWave - 1) smem[w] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t run = 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            int64_t t = smem[i];
            smem[i] = run;
            run += t;
        }
        smem[NW] = run;
    }
    __syncthreads();
    int64_t r = inc + smem[w];
    *total = smem[NW];
    __syncthreads();
    return r;
}

// Bit cast helpers for 16-bit types.
__device__ __forceinline__ float to_float(float v) { return v; }
__device__ __forceinline__ float to_float(_Float16 v) { return (float)v; }
__device__ __forceinline__ float to_float(__hip_bfloat16 v) { return __bfloat162float(v); }

template <typename T>
__device__ __forceinline__ T from_float(float v);
template <>
__device__ __forceinline__ float from_float<float>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 from_float<_Float16>(float v) { return (_Float16)v; }
template <>
__device__ __forceinline__ __hip_bfloat16 from_float<__hip_bfloat16>(float v) {
    return __float2bfloat16(v);  // round to nearest even
}

inline size_t dtype_size(int32_t dt) {
    switch (dt) {
        case GRWS_F32: return 4;
        case GRWS_F16: return 2;
        case GRWS_BF16: return 2;
        default: return 0;
    }
}

// ---------------------------------------------------------------------------
// device-wide scans (scan.hip)
// ---------------------------------------------------------------------------
// Exclusive (or inclusive) prefix sum over n int32 or int64 inputs into int64
// outputs.  When `exclusive_total` is non-null (exclusive mode), out has n+1
// entries and out[n] receives the total.  Workspace from scan_workspace_bytes.
size_t scan_workspace_bytes(int64_t n);
int scan_i32_to_i64(const int32_t* in, int64_t* out, int64_t n, bool inclusive, void* ws,
                    size_t ws_bytes, hipStream_t stream);
int scan_i64_to_i64(const int64_t* in, int64_t* out, int64_t n, bool inclusive, void* ws,
                    size_t ws_bytes, hipStream_t stream);

// Stable LSD radix sort of (u64 key, u32 payload) pairs over the low `bits`
// key bits (sort.hip).  The result lands in keys/vals or, when
// *result_in_alt, in keys_alt/vals_alt.
size_t radix_sort_workspace_bytes(int64_t n);
int radix_sort_pairs(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt, uint32_t* vals_alt, int64_t n, int bits,
                     void* ws, size_t ws_bytes, hipStream_t stream, bool* result_in_alt);

// Fill helpers (plain kernels: safe under graph capture, unlike memset nodes).
int fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t stream);
int fill_i64(int64_t* p, int64_t n, int64_t v, hipStream_t stream);
int fill_bytes_zero(void* p, size_t bytes, hipStream_t stream);

}  // namespace grws
