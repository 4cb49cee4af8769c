// ktimer.hpp -- per-kernel GPU timing, switched on by HYMT_HIP_TIMING=1 in the
// environment when a context is created (the HIP counterpart of the
// reference's HYMT_VK_TIMING / HYMT_VK_PFPROF timestamp modes,
// VulkanBackend.cs:55,71-74,410-411,488-540).
//
// Each public call of a timing context brackets its work in a TimedCall; every
// launcher brackets each kernel it enqueues in a KernelSpan.  A span made for
// one launch hands its event pair to that launch (launch() below, through
// hipExtLaunchKernelGGL), so the dispatch itself stamps the kernel's start and
// end, as a profiler's kernel trace does; other spans (a library call, a loop
// of launches, a graph replay) record an event before and after their work on
// the launch stream.  When the outermost
// TimedCall ends it waits for the last event and prints one line to stderr:
//   [hymt timing] <call>(<arg>): <span> us on the GPU, <n> kernels | <kernel> <count>x <us> | ...
// with the kernels summed by name, largest first.  hymt_destroy prints the
// totals over the context's life.  With timing off a KernelSpan costs one
// thread-local load; calls made while recording a graph are not timed.
// HYMT_HIP_TIMING=quiet collects the same totals without printing, for a
// caller that reads them (hymt_timing_get).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace hymt {

class KernelTimer;

// A timer when HYMT_HIP_TIMING is 1 or quiet, else null.
KernelTimer *timer_from_env();
// A timer that prints per call (print) or only collects.
KernelTimer *timer_create(bool print);
void timer_set_print(KernelTimer *t, bool print);
// Totals of `kernel` over the calls reported so far; false if never timed.
bool timer_totals(const KernelTimer *t, const char *kernel, long *count, double *us);
void timer_reset(KernelTimer *t);
// Prints the totals and releases the events; null is a no-op.
void timer_destroy(KernelTimer *t);

class TimedCall {
  public:
    TimedCall(KernelTimer *t, const char *call, long arg);  // t null: no-op
    ~TimedCall();
    TimedCall(const TimedCall &) = delete;
    TimedCall &operator=(const TimedCall &) = delete;

  private:
    KernelTimer *t_;
    KernelTimer *prev_;
};

class KernelSpan {
  public:
    // by_launch: the span's one kernel is enqueued with launch(span, ...)
    KernelSpan(const char *name, hipStream_t s, bool by_launch = false);
    ~KernelSpan();
    bool on() const { return rec_ >= 0; }
    hipEvent_t start() const;
    hipEvent_t stop() const;
    KernelSpan(const KernelSpan &) = delete;
    KernelSpan &operator=(const KernelSpan &) = delete;

  private:
    KernelTimer *t_;
    int rec_;
    hipStream_t s_;
    bool by_launch_;
};

// Enqueue `k` on `s`; with timing on, with the span's events stamped by the
// dispatch.  Calls being recorded into a graph are never timed, so they always
// take the plain launch.
template <typename K, typename... Args>
inline void launch(const KernelSpan &span, K k, dim3 grid, dim3 block, uint32_t lds, hipStream_t s,
                   Args... args) {
    if (span.on())
        hipExtLaunchKernelGGL(k, grid, block, lds, s, span.start(), span.stop(), 0, args...);
    else
        hipLaunchKernelGGL(k, grid, block, lds, s, args...);
}

}  // namespace hymt
