// ceilings.hip -- measured ceilings of one MI355X (gfx950), reported by
// bench.py beside the vendor peaks: the cost of a dependent kernel launch,
// the time to stream a buffer of a given size from HBM (the floor under a
// decode call of that many bytes), the cost of handing split partials to a
// merge (a second launch against a last-arriving workgroup in the same
// launch), the dense bf16 MFMA rate and the LDS read rate.  libhymt_ceilings.so is a measurement tool of the benchmark, not part
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

// Handing split partials to a merge, on a 4k-position decode call's shape: 4
// groups (kv heads) of 64 workgroups (splits), each streaming 32 KiB and
// writing a 2 KiB partial, then
//   MODE 0  nothing more (the split kernel alone);
//   MODE 1  plain stores; a second, dependent launch merges (merge_kernel);
//   MODE 2  device-coherent (sc1) stores, a device-scope ticket per group,
//           and the workgroup holding a group's last ticket merges its 64
//           partials with device-coherent loads in the same launch.
// The merge is a sum (its cost is the reads), written to out[group][512];
// `done` counts the in-kernel merges so the host can check that every call
// merged every group.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t hc_rsrc(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, 0x7fffffff, 0x00020000);
}
typedef unsigned hc_u4 __attribute__((ext_vector_type(4)));
template <int MODE>
__global__ __launch_bounds__(256) void split_kernel(const uint4 *src, float4 *part, unsigned *ticket, float4 *out,
                                                    unsigned *done) {
    const int grp = blockIdx.x & 3, idx = blockIdx.x >> 2, tid = threadIdx.x;
    const uint4 *p = src + (size_t)blockIdx.x * 2048 + tid;
    uint4 v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = p[256 * i];
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    const float f = (float)(x & 0xFFFF) * 1e-6f + (float)idx;
    __shared__ float4 red[128];
    __shared__ int last;
    float4 *pp = part + (size_t)(grp * 64 + idx) * 128;
    if (MODE != 2) {
        if (tid < 128) pp[tid] = make_float4(f, f, f, f);
        return;
    }
    const __amdgpu_buffer_rsrc_t r = hc_rsrc(part + (size_t)grp * 64 * 128);
    if (tid < 128) {
        const hc_u4 u = {__float_as_uint(f), __float_as_uint(f), __float_as_uint(f), __float_as_uint(f)};
        __builtin_amdgcn_raw_buffer_store_b128(u, r, (idx * 128 + tid) * 16, 0, 16);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(ticket + grp * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 63u;
    __syncthreads();
    if (!last) return;
    // 64 partials of 128 float4: thread (split parity h, float4 c), 32 loads at once
    const int c = tid & 127, h = tid >> 7;
    float4 a[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const hc_u4 u = __builtin_amdgcn_raw_buffer_load_b128(r, ((h + 2 * i) * 128 + c) * 16, 0, 16);
        a[i] = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
    }
    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < 32; i++) sum = make_float4(sum.x + a[i].x, sum.y + a[i].y, sum.z + a[i].z, sum.w + a[i].w);
    if (h) red[c] = sum;
    __syncthreads();
    if (!h) {
        const float4 b = red[c];
        out[grp * 128 + c] = make_float4(sum.x + b.x, sum.y + b.y, sum.z + b.z, sum.w + b.w);
    }
    if (tid == 0) {
        __hip_atomic_store(ticket + grp * 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(done + grp * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
// MODE 1's second launch: workgroup (group, 8-float4 slice); thread (split
// group of 32, float4 of the slice) sums two splits, then the 32 split
// groups through LDS
__global__ __launch_bounds__(256) void merge_kernel(const float4 *part, float4 *out) {
    const int grp = blockIdx.x >> 4, sl = blockIdx.x & 15, tid = threadIdx.x, f4 = tid & 7, sg = tid >> 3;
    const float4 *pp = part + (size_t)grp * 64 * 128 + sl * 8 + f4;
    const float4 a = pp[(size_t)sg * 128], b = pp[(size_t)(sg + 32) * 128];
    __shared__ float4 red[32][8];
    red[sg][f4] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    __syncthreads();
    if (tid < 8) {
        float4 s = red[0][tid];
        for (int g = 1; g < 32; g++) s = make_float4(s.x + red[g][tid].x, s.y + red[g][tid].y, s.z + red[g][tid].z, s.w + red[g][tid].w);
        out[grp * 128 + sl * 8 + tid] = s;
    }
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

// Microseconds per call of the split-partial handoff (split_kernel, MODE
// 0/1/2 above), calls back to back in a recorded graph, each over its own
// 8 MiB of inputs (> 1 GiB in all).  MODE 2 checks afterwards that every call
// merged every group (returns hipErrorUnknown otherwise).
int hc_handoff(int mode, double *us) {
    if (mode < 0 || mode > 2) return (int)hipErrorInvalidValue;
    constexpr int kWg = 256;
    const size_t buf_bytes = (size_t)kWg * 32768;
    const int nbuf = (int)(((size_t)1 << 30) / buf_bytes) + 1;
    Timer t;
    if (int e = t.init()) return e;
    std::vector<void *> bufs(nbuf, nullptr);
    float4 *part = nullptr, *out = nullptr;
    unsigned *ticket = nullptr, *done = nullptr;
    int rc = 0;
    for (int i = 0; i < nbuf && !rc; i++) {
        rc = (int)hipMalloc(&bufs[i], buf_bytes);
        if (!rc) rc = (int)hipMemsetAsync(bufs[i], i & 0xff, buf_bytes, t.s);
    }
    if (!rc) rc = (int)hipMalloc((void **)&part, (size_t)4 * 64 * 128 * 16);
    if (!rc) rc = (int)hipMalloc((void **)&out, (size_t)4 * 128 * 16);
    if (!rc) rc = (int)hipMalloc((void **)&ticket, 4 * 128);
    if (!rc) rc = (int)hipMalloc((void **)&done, 4 * 128);
    if (!rc) rc = (int)hipMemsetAsync(ticket, 0, 4 * 128, t.s);
    if (!rc) rc = (int)hipMemsetAsync(done, 0, 4 * 128, t.s);
    if (!rc) rc = (int)hipStreamSynchronize(t.s);
    const int reps = nbuf >= 32 ? 4 : 64 / nbuf + 1;
    if (!rc)
        rc = time_launches(t, nbuf, reps, true, [&](int i) {
            const uint4 *src = (const uint4 *)bufs[i];
            if (mode == 2) {
                hipLaunchKernelGGL(split_kernel<2>, dim3(kWg), dim3(256), 0, t.s, src, part, ticket, out, done);
            } else {
                hipLaunchKernelGGL(split_kernel<0>, dim3(kWg), dim3(256), 0, t.s, src, part, ticket, out, done);
                if (mode == 1) hipLaunchKernelGGL(merge_kernel, dim3(64), dim3(256), 0, t.s, part, out);
            }
        }, us);
    if (!rc && mode == 2) {
        unsigned h[4 * 32] = {};
        rc = (int)hipMemcpy(h, done, sizeof(h), hipMemcpyDeviceToHost);
        const unsigned calls = (unsigned)nbuf * (3 + reps);  // time_launches: 3 warm-up runs, then reps
        for (int g = 0; g < 4 && !rc; g++)
            if (h[g * 32] != calls) rc = (int)hipErrorUnknown;
    }
    for (void *b : bufs)
        if (b) (void)hipFree(b);
    for (void *b : {(void *)part, (void *)out, (void *)ticket, (void *)done})
        if (b) (void)hipFree(b);
    return rc;
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
