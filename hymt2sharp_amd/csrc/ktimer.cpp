// ktimer.cpp -- the HYMT_HIP_TIMING mode declared in ktimer.hpp.
#include "ktimer.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace hymt {

namespace {
thread_local KernelTimer *tl_active = nullptr;
}

class KernelTimer {
  public:
    struct Rec {
        const char *name;
        int e0, e1;
    };
    struct Total {
        long count = 0;
        double us = 0;
    };

    explicit KernelTimer(bool print) : print_(print) {}
    ~KernelTimer() {
        for (hipEvent_t e : pool_) (void)hipEventDestroy(e);
    }

    int event() {
        if (used_ == (int)pool_.size()) {
            hipEvent_t e = nullptr;
            if (hipEventCreate(&e) != hipSuccess) return -1;
            pool_.push_back(e);
        }
        return used_++;
    }
    hipEvent_t ev_start(int rec) const { return pool_[recs_[rec].e0]; }
    hipEvent_t ev_stop(int rec) const { return pool_[recs_[rec].e1]; }

    // record: stamp the start now (else the launch stamps both events)
    int begin_kernel(const char *name, hipStream_t s, bool record) {
        const int e0 = event(), e1 = event();
        if (e0 < 0 || e1 < 0 || (record && hipEventRecord(pool_[e0], s) != hipSuccess)) return -1;
        recs_.push_back({name, e0, e1});
        return (int)recs_.size() - 1;
    }
    void end_kernel(int rec, hipStream_t s) {
        if (rec >= 0 && hipEventRecord(pool_[recs_[rec].e1], s) != hipSuccess) recs_[rec].e1 = -1;
    }

    void begin_call(const char *call, long arg) {
        if (depth_++ > 0) return;
        call_ = call;
        arg_ = arg;
        recs_.clear();
        used_ = 0;
    }
    void end_call() {
        if (--depth_ > 0) return;
        report();
    }

    bool totals(const char *kernel, long *count, double *us) const {
        auto it = life_.find(kernel);
        if (it == life_.end()) return false;
        *count = it->second.count;
        *us = it->second.us;
        return true;
    }
    void reset() {
        life_.clear();
        calls_ = 0;
    }

    void set_print(bool p) { print_ = p; }

    void summary() const {
        if (calls_ == 0 || !print_) return;
        std::string line = "[hymt timing] totals over " + std::to_string(calls_) + " calls:";
        append_sorted(line, life_);
        std::fprintf(stderr, "%s\n", line.c_str());
        std::fflush(stderr);
    }

  private:
    static void append_sorted(std::string &line, const std::map<std::string, Total> &m) {
        std::vector<std::pair<std::string, Total>> v(m.begin(), m.end());
        std::sort(v.begin(), v.end(), [](const auto &a, const auto &b) { return a.second.us > b.second.us; });
        char buf[160];
        for (const auto &kv : v) {
            std::snprintf(buf, sizeof buf, " | %s %ldx %.1f us", kv.first.c_str(), kv.second.count, kv.second.us);
            line += buf;
        }
    }

    void report() {
        if (recs_.empty()) return;
        // the last event recorded is the last end event of the call
        int last = -1;
        for (const Rec &r : recs_)
            if (r.e1 >= 0) last = std::max(last, r.e1);
        if (last < 0 || hipEventSynchronize(pool_[last]) != hipSuccess) return;
        std::map<std::string, Total> per;
        float span = 0;
        (void)hipEventElapsedTime(&span, pool_[recs_.front().e0], pool_[last]);
        for (const Rec &r : recs_) {
            float ms = 0;
            if (r.e1 < 0 || hipEventElapsedTime(&ms, pool_[r.e0], pool_[r.e1]) != hipSuccess) continue;
            Total &t = per[r.name];
            t.count += 1;
            t.us += 1e3 * ms;
            Total &l = life_[r.name];
            l.count += 1;
            l.us += 1e3 * ms;
        }
        ++calls_;
        if (!print_) return;
        char head[160];
        std::snprintf(head, sizeof head, "[hymt timing] %s(%ld): %.1f us on the GPU, %zu kernels", call_, arg_,
                      1e3 * span, recs_.size());
        std::string line = head;
        append_sorted(line, per);
        std::fprintf(stderr, "%s\n", line.c_str());
        std::fflush(stderr);
    }

    std::vector<hipEvent_t> pool_;
    int used_ = 0;
    std::vector<Rec> recs_;
    int depth_ = 0;
    const char *call_ = "";
    long arg_ = 0;
    long calls_ = 0;
    std::map<std::string, Total> life_;
    bool print_;
};

KernelTimer *timer_from_env() {
    const char *v = std::getenv("HYMT_HIP_TIMING");
    if (!v) return nullptr;
    if (std::strcmp(v, "1") == 0) return new KernelTimer(true);
    if (std::strcmp(v, "quiet") == 0) return new KernelTimer(false);
    return nullptr;
}

KernelTimer *timer_create(bool print) { return new KernelTimer(print); }

void timer_set_print(KernelTimer *t, bool print) {
    if (t) t->set_print(print);
}

void timer_destroy(KernelTimer *t) {
    if (!t) return;
    t->summary();
    delete t;
}

bool timer_totals(const KernelTimer *t, const char *kernel, long *count, double *us) {
    return t && kernel && t->totals(kernel, count, us);
}

void timer_reset(KernelTimer *t) {
    if (t) t->reset();
}

TimedCall::TimedCall(KernelTimer *t, const char *call, long arg) : t_(t), prev_(tl_active) {
    if (!t_) return;
    tl_active = t_;
    t_->begin_call(call, arg);
}

TimedCall::~TimedCall() {
    if (!t_) return;
    t_->end_call();
    tl_active = prev_;
}

KernelSpan::KernelSpan(const char *name, hipStream_t s, bool by_launch)
    : t_(tl_active), rec_(-1), s_(s), by_launch_(by_launch) {
    if (t_) rec_ = t_->begin_kernel(name, s, !by_launch);
}

KernelSpan::~KernelSpan() {
    if (t_ && !by_launch_) t_->end_kernel(rec_, s_);
}

hipEvent_t KernelSpan::start() const { return rec_ >= 0 ? t_->ev_start(rec_) : nullptr; }
hipEvent_t KernelSpan::stop() const { return rec_ >= 0 ? t_->ev_stop(rec_) : nullptr; }

}  // namespace hymt
