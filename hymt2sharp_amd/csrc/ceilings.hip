// ceilings.hip -- measured ceilings of one MI355X (gfx950), reported by
// bench.py beside the vendor peaks: the cost of a dependent kernel launch,
// the time to stream a buffer of a given size from HBM (the floor under a
// decode call of that many bytes), the dense bf16 MFMA rate and the LDS read
// rate.  libhymt_ceilings.so is a measurement tool of the benchmark, not part
// of the attention path's C ABI.  Every function allocates what it times,
// times it with HIP events on its own stream and frees it; all return 0 on
// success or the hipError_t of the first failing call.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace {

#define CK(x)                                  \
    do {                                       \
        hipError_t e_ = (x);                   \
        if (e_ != hipSuccess) return (int)e_;  \
    } while (0)

__global__ void empty_kernel(int *sink) {
    if (sink && threadIdx.x == 1000000) sink[0] = 1;  // never true: keeps the argument live
}

// Each workgroup streams `per_wg` 16-byte vectors of src[blockIdx.x * per_wg
// ...]: every thread issues all its loads before using any (the access
// pattern of the decode kernel), then folds them; the fold is stored only if
// it equals a value no input produces, so nothing is written.
template <int PER_THREAD>
__global__ __launch_bounds__(256) void stream_kernel(const uint4 *src, uint32_t *sink, uint32_t never) {
    const uint4 *p = src + (size_t)blockIdx.x * (256 * PER_THREAD) + threadIdx.x;
    uint4 v[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; i++) v[i] = p[256 * i];
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < PER_THREAD; i++) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (x == never) sink[blockIdx.x] = x;
}

// Independent MFMA chains: each wave keeps 8 accumulators of
// v_mfma_f32_16x16x32_bf16 busy for `iters` rounds (16*16*32*2 FLOP each).
// The instructions are written out so that every accumulator stays in its
// registers (the compiler otherwise copies accumulators between rounds); the
// products are never used, only timed.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
#define HC_MFMA(c) asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b))
__global__ __launch_bounds__(256) void mfma_kernel(float *sink, int iters) {
    bf16x8 a, b;
    for (int i = 0; i < 8; i++) {
        a[i] = (__bf16)(float)(threadIdx.x & 7);
        b[i] = (__bf16)(float)((threadIdx.x >> 3) & 7);
    }
    f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0, c6 = c0, c7 = c0;
    for (int it = 0; it < iters; it++) {
        HC_MFMA(c0);
        HC_MFMA(c1);
        HC_MFMA(c2);
        HC_MFMA(c3);
        HC_MFMA(c4);
        HC_MFMA(c5);
        HC_MFMA(c6);
        HC_MFMA(c7);
    }
    const f32x4 s = c0 + c1 + c2 + c3 + c4 + c5 + c6 + c7;
    if (s[0] + s[1] + s[2] + s[3] == -1.0f) sink[blockIdx.x] = s[0];
}
#undef HC_MFMA

// LDS reads: every thread reads 16 bytes per step from a 64 KiB array, the
// lanes of a wave covering 1 KiB contiguously (no bank conflicts).
__global__ __launch_bounds__(256) void lds_kernel(uint32_t *sink, int iters) {
    __shared__ uint4 buf[4096];
    for (int i = threadIdx.x; i < 4096; i += 256) buf[i] = make_uint4(i, i + 1, i + 2, i + 3);
    __syncthreads();
    uint4 acc = make_uint4(0, 0, 0, 0);
    int idx = threadIdx.x;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint4 v = buf[(idx + 256 * k) & 4095];
            acc.x ^= v.x;
            acc.y += v.y;
            acc.z ^= v.z;
            acc.w += v.w;
        }
        idx += 64;
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) sink[blockIdx.x] = acc.x;
}

struct Timer {
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int init() {
        CK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        CK(hipEventCreate(&e0));
        CK(hipEventCreate(&e1));
        return 0;
    }
    ~Timer() {
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        if (s) (void)hipStreamDestroy(s);
    }
};

// Record `n` launches of `launch(i)` into a graph (or enqueue them eagerly)
// and time `reps` replays; returns microseconds per launch.
template <typename F> int time_launches(Timer &t, int n, int reps, bool graph, F launch, double *us) {
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    if (graph) {
        CK(hipStreamBeginCapture(t.s, hipStreamCaptureModeThreadLocal));
        for (int i = 0; i < n; i++) launch(i);
        CK(hipStreamEndCapture(t.s, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    }
    auto run = [&]() -> int {
        if (graph) {
            CK(hipGraphLaunch(ge, t.s));
        } else {
            for (int i = 0; i < n; i++) launch(i);
            CK(hipGetLastError());
        }
        return 0;
    };
    for (int r = 0; r < 3; r++)
        if (int e = run()) return e;
    CK(hipStreamSynchronize(t.s));
    CK(hipEventRecord(t.e0, t.s));
    for (int r = 0; r < reps; r++)
        if (int e = run()) return e;
    CK(hipEventRecord(t.e1, t.s));
    CK(hipEventSynchronize(t.e1));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, t.e0, t.e1));
    *us = (double)ms * 1e3 / ((double)n * reps);
    if (ge) CK(hipGraphExecDestroy(ge));
    if (g) CK(hipGraphDestroy(g));
    return 0;
}

}  // namespace

extern "C" {

// Microseconds per launch of an empty one-wave kernel, back to back on one
// stream (each waits for the previous: the stream's in-order rule), in a
// recorded graph of 32 launches (graph != 0) or enqueued one by one.
int hc_launch_gap(int graph, double *us) {
    Timer t;
    if (int e = t.init()) return e;
    return time_launches(t, 32, 200, graph != 0, [&](int) {
        hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, t.s, nullptr);
    }, us);
}

// Microseconds per launch of a kernel streaming `bytes` (rounded to whole
// workgroups of 256 threads x per_thread 16-byte loads: per_thread 4, 8, 16
// or 32, i.e. 16 to 128 KiB per workgroup) from HBM, back to back over
// distinct buffers -- enough of them (> 1 GiB in all, at least 2) that the
// 256 MiB MALL cannot serve the reads -- recorded as one graph (graph != 0)
// or enqueued one by one.  *wgs receives the grid size.
int hc_stream_read(size_t bytes, int per_thread, int graph, double *us, int *wgs) {
    if (per_thread != 4 && per_thread != 8 && per_thread != 16 && per_thread != 32) return (int)hipErrorInvalidValue;
    const size_t WG_BYTES = (size_t)256 * per_thread * 16;
    const int nwg = (int)((bytes + WG_BYTES - 1) / WG_BYTES);
    const size_t buf_bytes = (size_t)nwg * WG_BYTES;
    int nbuf = (int)(((size_t)1 << 30) / buf_bytes) + 1;
    if (nbuf < 2) nbuf = 2;
    Timer t;
    if (int e = t.init()) return e;
    std::vector<void *> bufs(nbuf, nullptr);
    uint32_t *sink = nullptr;
    int rc = 0;
    for (int i = 0; i < nbuf && !rc; i++) {
        rc = (int)hipMalloc(&bufs[i], buf_bytes);
        if (!rc) rc = (int)hipMemsetAsync(bufs[i], i & 0xff, buf_bytes, t.s);
    }
    if (!rc) rc = (int)hipMalloc((void **)&sink, (size_t)nwg * 4);
    if (!rc) rc = (int)hipStreamSynchronize(t.s);
    if (!rc)
        rc = time_launches(t, nbuf, nbuf >= 32 ? 4 : 64 / nbuf + 1, graph != 0, [&](int i) {
            const uint4 *src = (const uint4 *)bufs[i];
            switch (per_thread) {
            case 4: hipLaunchKernelGGL(stream_kernel<4>, dim3(nwg), dim3(256), 0, t.s, src, sink, 0x9e3779b9u); break;
            case 8: hipLaunchKernelGGL(stream_kernel<8>, dim3(nwg), dim3(256), 0, t.s, src, sink, 0x9e3779b9u); break;
            case 16: hipLaunchKernelGGL(stream_kernel<16>, dim3(nwg), dim3(256), 0, t.s, src, sink, 0x9e3779b9u); break;
            default: hipLaunchKernelGGL(stream_kernel<32>, dim3(nwg), dim3(256), 0, t.s, src, sink, 0x9e3779b9u);
            }
        }, us);
    for (void *b : bufs)
        if (b) (void)hipFree(b);
    if (sink) (void)hipFree(sink);
    if (rc) return rc;
    *wgs = nwg;
    return 0;
}

// Dispatch-stamped duration (hipExtLaunchKernelGGL's start/stop events, what
// the library's timing mode and rocprofv3's kernel trace report) of an empty
// one-wave kernel (kind 0) or of a kernel streaming `bytes` from HBM with the
// decode kernel's pattern (kind 1, 16 KiB per workgroup, a fresh buffer per
// launch), averaged over 64 launches, each alone on the stream (isolated:
// the stream drained before it, as in a call timed by itself) or back to
// back.  Microseconds.
int hc_dispatch_duration(int kind, size_t bytes, int isolated, double *us) {
    constexpr int kN = 64, kPer = 4;
    const size_t WG_BYTES = (size_t)256 * kPer * 16;
    const int nwg = kind ? (int)((bytes + WG_BYTES - 1) / WG_BYTES) : 1;
    Timer t;
    if (int e = t.init()) return e;
    std::vector<void *> bufs(kind ? kN : 0, nullptr);
    std::vector<hipEvent_t> ev(2 * kN, nullptr);
    uint32_t *sink = nullptr;
    int rc = (int)hipMalloc((void **)&sink, (size_t)nwg * 4);
    for (size_t i = 0; i < bufs.size() && !rc; i++) {
        rc = (int)hipMalloc(&bufs[i], (size_t)nwg * WG_BYTES);
        if (!rc) rc = (int)hipMemsetAsync(bufs[i], (int)i & 0xff, (size_t)nwg * WG_BYTES, t.s);
    }
    for (int i = 0; i < 2 * kN && !rc; i++) rc = (int)hipEventCreate(&ev[i]);
    if (!rc) rc = (int)hipStreamSynchronize(t.s);
    for (int rep = 0; rep < 2 && !rc; rep++) {  // the first round warms up
        for (int i = 0; i < kN && !rc; i++) {
            if (isolated) rc = (int)hipStreamSynchronize(t.s);
            if (rc) break;
            if (kind)
                hipExtLaunchKernelGGL(stream_kernel<kPer>, dim3(nwg), dim3(256), 0, t.s, ev[2 * i], ev[2 * i + 1], 0,
                                      (const uint4 *)bufs[i], sink, 0x9e3779b9u);
            else
                hipExtLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, t.s, ev[2 * i], ev[2 * i + 1], 0, (int *)sink);
            rc = (int)hipGetLastError();
        }
        if (!rc) rc = (int)hipStreamSynchronize(t.s);
    }
    double sum = 0.0;
    for (int i = 0; i < kN && !rc; i++) {
        float ms = 0.f;
        rc = (int)hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]);
        sum += ms;
    }
    for (hipEvent_t e : ev)
        if (e) (void)hipEventDestroy(e);
    for (void *b : bufs)
        if (b) (void)hipFree(b);
    if (sink) (void)hipFree(sink);
    if (rc) return rc;
    *us = sum * 1e3 / kN;
    return 0;
}

// Dense bf16 MFMA rate (TFLOP/s) with `waves_per_simd` waves on every SIMD of
// every CU (grid = CUs x waves_per_simd workgroups of 4 waves).
int hc_mfma_bf16(int waves_per_simd, double *tflops) {
    int dev = 0, cus = 0;
    CK(hipGetDevice(&dev));
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    Timer t;
    if (int e = t.init()) return e;
    float *sink = nullptr;
    CK(hipMalloc((void **)&sink, 4 * 4096));
    const int iters = 4096, nwg = cus * waves_per_simd;
    double us = 0.0;
    int rc = time_launches(t, 1, 10, false, [&](int) {
        hipLaunchKernelGGL(mfma_kernel, dim3(nwg), dim3(256), 0, t.s, sink, iters);
    }, &us);
    (void)hipFree(sink);
    if (rc) return rc;
    const double flops = (double)nwg * 4 * iters * 8 * (16.0 * 16 * 32 * 2);
    *tflops = flops / (us * 1e-6) / 1e12;
    return 0;
}

// LDS read rate (TB/s over the whole chip), one 256-thread workgroup per CU
// x `wgs_per_cu`, 16-byte conflict-free reads.
int hc_lds_read(int wgs_per_cu, double *tbs) {
    int dev = 0, cus = 0;
    CK(hipGetDevice(&dev));
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    Timer t;
    if (int e = t.init()) return e;
    uint32_t *sink = nullptr;
    CK(hipMalloc((void **)&sink, 4 * 4096));
    const int iters = 8192, nwg = cus * wgs_per_cu;
    double us = 0.0;
    int rc = time_launches(t, 1, 10, false, [&](int) {
        hipLaunchKernelGGL(lds_kernel, dim3(nwg), dim3(256), 0, t.s, sink, iters);
    }, &us);
    (void)hipFree(sink);
    if (rc) return rc;
    const double bytes = (double)nwg * 256 * iters * 8 * 16;
    *tbs = bytes / (us * 1e-6) / 1e12;
    return 0;
}

int hc_device_info(int *cus, int *clock_khz, int *mem_clock_khz, int *bus_bits) {
    int dev = 0;
    CK(hipGetDevice(&dev));
    CK(hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev));
    CK(hipDeviceGetAttribute(clock_khz, hipDeviceAttributeClockRate, dev));
    CK(hipDeviceGetAttribute(mem_clock_khz, hipDeviceAttributeMemoryClockRate, dev));
    CK(hipDeviceGetAttribute(bus_bits, hipDeviceAttributeMemoryBusWidth, dev));
    return 0;
}

}  // extern "C"
